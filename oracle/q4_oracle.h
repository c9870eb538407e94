/*
 * CPU oracle for the MLX-affine Q4/g64 quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: the tests, the smoke
 * check and the CPU-baseline leg of the benchmark load it to produce expected
 * values. Nothing on the product path (the HIP library under hyperion_amd/)
 * links, loads or calls it.
 *
 * Every function restates the arithmetic of MLX 0.32.0 (the third-party
 * library the reference calls; pinned at native/hyperion_mlx/CMakeLists.txt:17,
 * oracle/pyproject.toml:6-9, commit 7a1d4f5c per
 * docs/research/0001-m0-vendor-verification.md:8). MLX is not vendored in the
 * reference, so the restatements follow MLX's published algorithm and are
 * anchored on the reference's call sites:
 *   quantize      crates/hyperion-model/fixtures/build_gemma4_unified_tiny.py:54-57
 *   dequantize    native/hyperion_mlx/src/weights_loader.cc:53-69
 *   qmatmul       native/hyperion_mlx/src/weights.h:26-37, forward.cc:137-152
 *   gelu_tanh     native/hyperion_mlx/src/forward.cc:324-343
 *   softcap       native/hyperion_mlx/src/forward.cc:154-160
 *   embed scale   native/hyperion_mlx/src/forward.cc:126-131
 *   greedy sample native/hyperion_mlx/src/forward.cc:162-189 (the reference's own loop,
 *                 not MLX)
 *
 * Pinning status (what checks each function; see tests/test_oracle.py):
 *   orc_bf16_from_f32       pinned: numpy float32 -> bfloat16 RNE bit patterns computed
 *                           independently in the test, plus special values.
 *   orc_quantize_q4g64      pinned: the reference's tiny fixture (42 Q4 tensors,
 *                           19,456 groups) - dequant->requant round trip reproduces the
 *                           fixture's (q, scale, bias) bit-exactly on every group that
 *                           holds q=15; sign/zero-point invariants on all groups;
 *                           closed-form cases (exact grids, constant and zero groups).
 *   orc_dequantize_q4g64    pinned: mode 1 (one rounding, bf16(s*q + b)) is MLX's - the
 *                           reference's 12B embed golden (12b_hidden_golden.safetensors
 *                           'embed', forward_12b_test.cc:218) fits it in all 600 groups and
 *                           the op-composed mode 0 alone in none; mode 1 reproduces that
 *                           golden bit for bit from the Q4 rows recovered from it
 *                           (tests/test_golden_embed.py). Also exact values (power-of-two
 *                           scales, bias grids) and the fixture round trip. Mode 0 is kept
 *                           only to show the difference (38% of the decode weights).
 *   orc_qmatmul_f64         pinned: closed-form known-answer cases and brute force.
 *   orc_qmatmul_deq_f64     pinned: equals orc_qmatmul_f64 wherever the dequantized
 *                           weights are exact in bf16, and brute force over
 *                           orc_dequantize_q4g64 output.
 *   orc_qmatmul_f32_grouped pinned: exact-arithmetic known-answer cases (every partial
 *                           sum representable) and against orc_qmatmul_f64.
 *   orc_qmatmul_mlx_cpu     parity unpinned: restates MLX's scalar CPU loop with
 *                           bf16-typed accumulation; only an MLX import could pin that
 *                           MLX runs this loop. The loop as restated is pinned: its
 *                           per-element step equals an exact-rational evaluation of
 *                           dq = bf16(bf16(s*q) + b), sum = bf16(sum + bf16(x*dq)) on
 *                           small cases, and the bf16 sum stalls at 256 when adding 1.
 *                           Used only to report the reference-side error and the CPU
 *                           baseline.
 *   orc_gelu_tanh_mul_bf16  pinned bit-exactly over all 65,536 bf16 inputs against an
 *                           exact-arithmetic evaluation of the reference's op order
 *                           (fp32 result of each op rounded to bf16, tanh from fp64),
 *                           except the inputs whose tanh lies within 2^-20 of a bf16
 *                           rounding boundary (counted, under 200).
 *   orc_softcap_bf16        pinned likewise over all bf16 inputs, caps 30 and 50.
 *   orc_qmatmul_mlx_cpu_mt  pinned to orc_qmatmul_mlx_cpu: bit-identical outputs.
 *   orc_rms_norm_bf16       pinned: against the fp64 closed form within one bf16 rounding
 *                           (two with a weight) plus fp32 statistics, power-of-two weights
 *                           exactly, constant rows, and the weightless form equal to a
 *                           weight of ones. The summation order is the HIP kernels' own:
 *                           MLX's (its Metal simd reductions) is parity unpinned.
 *   orc_rope_bf16           pinned: position 0 and the unrotated pairs are the identity;
 *                           the fp64 rotation of the closed form (theta = pos * base^(-2i/D))
 *                           within bf16 rounding; the pairs (i, i + D/2) and the rotation's
 *                           sign checked on one-hot inputs; pair norms preserved. MLX's
 *                           metal::fast trigonometry is parity unpinned.
 *   orc_attention_f64       pinned: the softmax weights of a query sum to one; a single
 *                           visible key returns its value row; equal keys average the
 *                           values; the masks against brute-force position tests; GQA head
 *                           sharing; against numpy's dense fp64 attention on random cases.
 *   orc_sample_topk_bf16    pinned: against std::partial_sort with the reference's own
 *                           comparator (oracle/stl_partial_sort.cc, libstdc++) - the same
 *                           ids where the top k + 1 values are distinct, the same values
 *                           always; ties and NaN ordered as stated (partial_sort leaves
 *                           them unspecified) and checked on hand cases; top-1 and top-2
 *                           agree with orc_sample_greedy_bf16.
 *   orc_det_exp             pinned: within 2 ulp of the correctly rounded exp over a dense
 *                           sweep of (-86, 0]; exp(0) = 1 exactly; 0 at and below -86.
 *   orc_sample_stochastic_bf16
 *                           pinned against oracle/stl_sample_stochastic.cc, a restatement of
 *                           the reference's host algorithm (std::exp, std::sort,
 *                           std::partial_sort, std::mt19937_64 and uniform_real_distribution
 *                           from libstdc++): the same kept sets wherever no two kept/dropped
 *                           probabilities tie at a filter's boundary, the same token wherever
 *                           u is not within rounding of a running-sum boundary; the kept set
 *                           against a float64 numpy sort; the token frequencies against the
 *                           filtered softmax by a chi-square test; top_k = 1 and tiny
 *                           temperatures equal the greedy token; the non-finite rows as the
 *                           reference's arithmetic gives them. The summation orders are the
 *                           HIP kernels' own (the reference's are not fixed by its contract).
 *   orc_sample_greedy_bf16  pinned: against the definition computed independently with
 *                           numpy (first index of the maximum over non-NaN values, the
 *                           largest other value) on random rows with planted ties, NaN
 *                           and infinities, and hand cases (empty, all -inf, all NaN).
 */
#ifndef HYPERION_Q4_ORACLE_H
#define HYPERION_Q4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint16_t orc_bf16_from_f32(float f);
float orc_f32_from_bf16(uint16_t h);
void orc_bf16_from_f32_array(const float* in, int64_t n, uint16_t* out);
void orc_f32_from_bf16_array(const uint16_t* in, int64_t n, float* out);

/* mx.quantize(w, group_size=64, bits=4, mode="affine") on a bf16 [n, k] matrix. */
void orc_quantize_q4g64(const uint16_t* w, int64_t n, int64_t k,
                        uint32_t* wq, uint16_t* scales, uint16_t* biases);

/* mx.dequantize(..., dtype=bfloat16) of rows `rows[0..n_rows)` (rows==NULL: 0..n_rows).
 * mode 1: bf16(s*q + b)        (fp32 math, single rounding to bf16: MLX's dequantize)
 * mode 0: bf16(bf16(s*q) + b)  (op-composed, one rounding per op; not MLX's) */
void orc_dequantize_q4g64(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                          const uint32_t* rows, int64_t n_rows, int64_t k, int mode,
                          uint16_t* out);

/* Ground truth: y[m,n] = sum_k x[m,k] * (s*q + b), all in fp64. */
void orc_qmatmul_f64(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                     const uint16_t* biases, int64_t m, int64_t n, int64_t k, double* y);

/* y[m,n] = sum_k x[m,k] * W~[n,k] in fp64, where W~ is the bf16 dequantization of
 * orc_dequantize_q4g64 in `mode` (the weight values a bf16 MFMA GEMM consumes). */
void orc_qmatmul_deq_f64(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                         const uint16_t* biases, int64_t m, int64_t n, int64_t k, int mode,
                         double* y);

/* fp32, per group g: acc += s_g * sum(x*q) + b_g * sum(x), sequential order. */
void orc_qmatmul_f32_grouped(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                             const uint16_t* biases, int64_t m, int64_t n, int64_t k, float* y);

/* Restatement of MLX's scalar CPU quantized_matmul (transpose=true) with the
 * accumulator typed as the input dtype (bf16): every multiply/add rounds to bf16. */
void orc_qmatmul_mlx_cpu(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                         const uint16_t* biases, int64_t m, int64_t n, int64_t k, uint16_t* y);

/* ForwardPass::sample_greedy on one row of n bf16 logits: token, its logit, near_tie. */
void orc_sample_greedy_bf16(const uint16_t* logits, int64_t n, uint32_t* token, float* logit,
                            int32_t* near_tie);

/* The greedy epilogue's top-k sidecar (model.cc:278-288) of one row of n bf16 logits:
 * ids/values of the min(k, n) first elements in the order larger value, lower index,
 * NaN last; returns that count, zero-fills ids/values up to k. */
uint32_t orc_sample_topk_bf16(const uint16_t* logits, int64_t n, uint32_t k, uint32_t* ids, float* values);

/* exp(x) for x <= 0 as the sampling kernels compute it (0 at or below -86). */
float orc_det_exp(float x);

/* ForwardPass::sample_stochastic's draw (forward.cc:225-301) over one row of vocab bf16
 * logits with the defined orders of the HIP kernels: token and its logit; *kept (if non-null)
 * receives the size of the kept prefix (0 for rows drawn without weights). canon is the
 * uniform in [0, 1) the draw scales by the kept total. */
void orc_sample_stochastic_bf16(const uint16_t* logits, uint32_t vocab, float inv_temp, float top_p, float min_p,
                                int32_t top_k, float canon, uint32_t* token, float* logit, uint32_t* kept);

/* orc_qmatmul_mlx_cpu with output rows spread over `threads` OpenMP threads
 * (bit-identical result; the multi-core CPU baseline). */
void orc_qmatmul_mlx_cpu_mt(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                            const uint16_t* biases, int64_t m, int64_t n, int64_t k, int threads,
                            uint16_t* y);

/* Rows [n0, n1) only of orc_qmatmul_mlx_cpu (bounded CPU-baseline samples). */
void orc_qmatmul_mlx_cpu_rows(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                              const uint16_t* biases, int64_t m, int64_t n0, int64_t n1,
                              int64_t k, uint16_t* y);

/* gelu_tanh(gate) * up as the reference's chain of bf16-rounded ops. */
void orc_gelu_tanh_mul_bf16(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* out);
void orc_gelu_tanh_bf16(const uint16_t* x, int64_t n, uint16_t* out);

/* softcap: bf16(bf16(tanh(bf16(x / cap))) * cap) with cap rounded to bf16. */
void orc_softcap_bf16(const uint16_t* x, int64_t n, float cap, uint16_t* out);

/* Elementwise bf16 multiply by a bf16 constant (embed scale). */
void orc_scale_bf16(const uint16_t* x, int64_t n, float c, uint16_t* out);

/* mx::fast::rms_norm with the HIP kernels' summation order; w may be NULL. */
void orc_rms_norm_bf16(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t k, float eps, uint16_t* y);
/* mx::fast::rope, non-traditional, on x [rows, heads, head_dim] at positions offset + r. */
void orc_rope_bf16(const uint16_t* x, int64_t rows, int64_t heads, int64_t head_dim, int64_t rotated,
                   double base, int64_t offset, uint16_t* y);

/* Scaled dot-product attention of ForwardPass::attention (scale 1, causal + optional
 * sliding window, grouped-query heads) in fp64 over a cache prefix and a chunk. */
void orc_attention_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* cache_k,
                       const uint16_t* cache_v, int64_t cap, int64_t L, int64_t n_heads, int64_t n_kv,
                       int64_t d, int64_t offset, int64_t prefix_len, int64_t window, double* out);

#ifdef __cplusplus
}
#endif

#endif
