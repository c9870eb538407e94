// Host-side launchers of the gfx950 kernels. All pointers are device pointers,
// all launches are asynchronous on `stream`. Callers validate shapes first.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "hyperion_hip.h"

namespace hyperion::hip {

// A Q4/g64 projection [n, k]. w/scales/biases: MLX layout, codes uint32 [n, k/8],
// scales and biases bf16 [n, k/64] (native/hyperion_mlx/src/weights.h:18-25).
// codes/sb: the tiled resident layout of q4_layout.h (null when not resident).
struct Q4Matrix {
    const uint32_t* w = nullptr;
    const uint16_t* scales = nullptr;
    const uint16_t* biases = nullptr;
    uint32_t n = 0;
    uint32_t k = 0;
    const uint4* codes = nullptr;
    const uint2* sb = nullptr;
};

// MLX layout -> tiled layout (q4_layout.h), and back. Device pointers; the tiled
// buffers hold TiledDims::of(n, k).code_bytes() and .sb_bytes().
void launch_q4_tile(const uint32_t* w, const uint16_t* s, const uint16_t* b, uint32_t n, uint32_t k, uint4* codes,
                    uint2* sb, hipStream_t stream);
void launch_q4_untile(const uint4* codes, const uint2* sb, uint32_t n, uint32_t k, uint32_t* w, uint16_t* s,
                      uint16_t* b, hipStream_t stream);

enum class Epilogue : int {
    kNone = 0,
    kSoftcap = 1,   // y = softcap(bf16(acc)), forward.cc:154-160
};

// Largest m the skinny MFMA kernel handles, and the most projections one grouped
// launch covers.
constexpr uint32_t kSkinnyMaxM = 4;
constexpr uint32_t kSkinnyMaxGroup = 3;

// Skinny quantized matmul on MFMA (m <= kSkinnyMaxM) over the tiled layout:
// y[m, n] = x[m, k] . dequant(W)^T. With `up` non-null it is the fused gate/up:
// y = gelu_chain(x.G^T) * (x.U^T). `splits` waves share each 16-row tile (1, 2, 4, 8
// or 16; 1, 2 or 4 with the softcap epilogue; 0 chooses); ceil(k / 128) >= splits.
void launch_q4_skinny(const Q4Matrix& w, const Q4Matrix* up, const uint16_t* x, uint32_t m, uint16_t* y,
                      Epilogue epi, float cap_bf16, uint32_t splits, hipStream_t stream);
// One launch over `count` projections that share x (and k), e.g. q, k and v:
// ys[i][m, n_i] = x . dequant(W_i)^T. With rms_eps non-null each x row is first
// rms-normalised (q4_rmsnorm.h; the same bits as launch_rms_normalize with norm_w) in LDS;
// norm_w is the norm's bf16 weight [k] or null.
// With res non-null (and rms_eps), the rows normalised are the sandwich's output x =
// bf16(res->in + rms_norm(res->branch, res->w)) (times *res->scalar when non-null) - the
// bits of launch_residual_norm - written to res->out by one workgroup; x is unused.
struct SkinnyResidual {
    const uint16_t* branch;   // [m][k]
    const uint16_t* in;       // [m][k], the residual stream
    uint16_t* out;            // [m][k], the updated residual stream (not `in`)
    const uint16_t* w;        // [k] the branch's post-norm weight
    const uint16_t* scalar;   // bf16 [1] or null
};
void launch_q4_skinny_group(const Q4Matrix* const* ws, uint16_t* const* ys, uint32_t count, const uint16_t* x,
                            uint32_t m, const float* rms_eps, const uint16_t* norm_w, hipStream_t stream,
                            const SkinnyResidual* res = nullptr);
// Whether launch_q4_skinny_group takes a residual at (m, k): every unit held by one thread.
bool skinny_resid_supported(uint32_t m, uint32_t k);
// Splits for `tiles` 16-row tiles, `pairs` group pairs and m rows of one launch form,
// and whether (m, k) fits the kernel's LDS staging.
enum class SkinnyForm : int {
    kPlain = 0,   // one projection or a q/k/v group (optionally normalising)
    kDual = 1,    // the fused gate/up
    kHead = 2,    // the softcap LM head
};
uint32_t choose_skinny_splits(uint32_t tiles, uint32_t pairs, uint32_t m, SkinnyForm form);
bool skinny_supported(uint32_t m, uint32_t k, bool dual);
bool skinny_norm_supported(uint32_t m, uint32_t k);

// Prefill GEMM on bf16 MFMA over the tiled layout: Q4 codes dequantized in registers,
// x tiles in LDS. Plain bf16 output; epilogues for larger m run as the elementwise
// kernels below.
void launch_q4_gemm(const Q4Matrix& w, const uint16_t* x, uint32_t m, uint16_t* y, hipStream_t stream);
// y = bf16(gelu_chain(x . G^T) * (x . U^T)) as one dual GEMM: each wave accumulates a gate
// tile and the same up tile, the epilogue applies the gating. Same kernel, split and sums
// as the grouped GEMM of [gate, up], so y is the GELU chain over that launch's outputs bit
// for bit.
void launch_q4_gemm_gate_up(const Q4Matrix& gate, const Q4Matrix& up, const uint16_t* x, uint32_t m, uint16_t* y,
                            hipStream_t stream);
// launch_q4_gemm with the split-k partials in a fixed device scratch array instead of a
// stream-ordered temporary: allocates nothing (INVALID_ARGUMENT if the call's partials
// exceed the 64 MiB scratch). Calls on one device share the scratch.
void launch_q4_gemm_noalloc(const Q4Matrix& w, const uint16_t* x, uint32_t m, uint16_t* y, hipStream_t stream);
// One launch over `count` (<= 3) projections that share x and k (q, k and v):
// ys[i][m, n_i] = x . dequant(W_i)^T.
void launch_q4_gemm_group(const Q4Matrix* const* ws, uint16_t* const* ys, uint32_t count, const uint16_t* x,
                          uint32_t m, hipStream_t stream);
// y = softcap(y) over `count` bf16 elements (in place).
void launch_softcap(uint16_t* y, float cap_bf16, uint64_t count, hipStream_t stream);
// y[r] = bf16(w * bf16(x[r] / sqrt(mean(x[r]^2) + eps))) for each of m rows of k bf16,
// w the bf16 weight [k] or null (then y = bf16(x / ...)); y may equal x.
void launch_rms_normalize(const uint16_t* x, const uint16_t* w, uint32_t m, uint32_t k, float eps, uint16_t* y,
                          hipStream_t stream);

// mx::fast::rope (non-traditional) of x [rows, heads, head_dim] at positions offset + r:
// pairs (i, i + head_dim/2) with i < rotated/2 rotate, the rest are copied (y may equal x).
void launch_rope(const uint16_t* x, uint32_t rows, uint32_t heads, uint32_t head_dim, uint32_t rotated, float base,
                 uint32_t offset, uint16_t* y, hipStream_t stream);

// ForwardPass::sample_greedy over each of `rows` rows of `vocab` bf16 logits -> out[row],
// with slice states in `workspace` (device memory of sample_greedy_workspace_bytes(),
// used by one stream at a time).
size_t sample_greedy_workspace_bytes();
void launch_sample_greedy(const uint16_t* logits, uint32_t rows, uint32_t vocab, HypGreedySample* out,
                          void* workspace, size_t workspace_bytes, hipStream_t stream);

// The greedy epilogue's top-k sidecar (plus the greedy fields) of each row -> out[row];
// same workspace as launch_sample_greedy; vocab <= sample_topk_max_vocab() (2^23).
constexpr uint32_t kHypTopK = HYP_TOP_K_LOGPROBS;
uint32_t sample_topk_max_vocab();
void launch_sample_topk(const uint16_t* logits, uint32_t rows, uint32_t vocab, HypTopKSample* out, void* workspace,
                        size_t workspace_bytes, hipStream_t stream);

// Temperature sampling of one row (ForwardPass::sample_stochastic, forward.cc:192-310), the
// filters and draw on the device. Its parameters live in device memory so that a captured
// decode step can sample with the configuration and uniforms the host writes before the
// replays: each launch draws with uniform[min(step, n_uniform - 1)] and advances step.
constexpr uint32_t kMaxSampledSteps = 256;
struct SampleParams {
    float inv_temp;   // 1 / temperature (fp32)
    float top_p;      // (0, 1]: nucleus; otherwise off
    float min_p;      // (0, 1): min-p; otherwise off
    int32_t top_k;    // (0, vocab): top-k; otherwise off
    uint32_t n_uniform;
    uint32_t step;
    float uniform[kMaxSampledSteps];   // std::generate_canonical<float> of std::mt19937_64, per step
};
// Device workspace of launch_sample_stochastic (256-byte aligned): 65536 value bins and a flag
// word, zero between launches (init_sample_stochastic_workspace clears a new workspace once;
// every launch leaves them zero), the decision of the cut, and the SampleParams.
size_t sample_stochastic_workspace_bytes();
void init_sample_stochastic_workspace(void* workspace, hipStream_t stream);
SampleParams* sample_stochastic_params(void* workspace);
// Write a one-draw SampleParams (uniform[0] = canon) into the workspace, as a kernel (its
// values travel as kernel arguments, so a captured call keeps them).
void launch_sample_params(void* workspace, float inv_temp, float top_p, float min_p, int32_t top_k, float canon,
                          hipStream_t stream);
// out->token_id, logit and near_tie (0) of the draw with the workspace's SampleParams; the
// top-k sidecar is launch_sample_topk's. vocab is at most 2^23.
void launch_sample_stochastic(const uint16_t* logits, uint32_t vocab, void* workspace, size_t workspace_bytes,
                              HypTopKSample* out, hipStream_t stream);

// Attention (forward.cc:376-508) over a KV cache prefix and the current chunk; see
// attention.hip. Decode splits the keys; the partial sums need attention_workspace_bytes.
constexpr uint32_t kAttnMaxSplits = 64;
struct AttnPrepareArgs;
struct AttnArgs {
    const uint16_t* q;         // [L][n_heads][head_dim]
    const uint16_t* k;         // [L][n_kv_heads][head_dim] (the chunk); null: the chunk is
    const uint16_t* v;         // already in the cache at positions offset .. offset + L - 1
    const uint16_t* cache_k;   // [cap][n_kv_heads][head_dim]
    const uint16_t* cache_v;
    uint16_t* out;             // [L][n_heads][head_dim]
    uint32_t L, n_heads, n_kv_heads, head_dim, cap, offset, prefix_len, window;
    void* workspace;
    size_t workspace_bytes;
    // Graph-replay form: with pos non-null the kernel reads the offset from *pos and takes
    // prefix_len = min(window, offset) (window > 0) or offset; the keys are split over
    // fixed_splits workgroups per kv head whatever the offset.
    const uint32_t* pos = nullptr;
    uint32_t fixed_splits = 1;
    // With prep non-null (one token, k = v = null, the decode form, a RoPE table): q is the
    // raw projection (prep->q, not modified) and the launch does launch_attn_prepare's work
    // itself, with its arithmetic: the query rows normalised and rotated per wave, and the
    // new token's K/V written to its cache slot by the wave whose keys hold it.
    const AttnPrepareArgs* prep = nullptr;
};
size_t attention_workspace_bytes(uint32_t n_kv_heads, uint32_t head_dim);
// The workspace with which launch_attention also splits the keys of chunks of up to max_L
// tokens (0 when no such chunk splits); with less it runs those chunks unsplit.
size_t attention_chunk_workspace_bytes(uint32_t max_L, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim);
uint32_t attention_splits(uint32_t L, uint32_t n_heads, uint32_t n_kv_heads, uint32_t keys);
// Whether AttnArgs::prep can fold the prepare for this geometry: one token runs the decode
// form (G <= 16 query rows per kv head) and the G query rows and the new K and V of one kv
// head fit one wave as 64-value units ((G + 2) * head_dim / 64 <= 64).
bool attention_prep_fits(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim);
void launch_attention(const AttnArgs& a, hipStream_t stream);
// Tokens pos0.. of k/v [n][n_kv_heads][head_dim] into cache slots (pos % cap).
void launch_kv_write(const uint16_t* k, const uint16_t* v, uint16_t* ck, uint16_t* cv, uint32_t n, uint32_t pos0,
                     uint32_t cap, uint32_t n_kv_heads, uint32_t head_dim, hipStream_t stream);

// q/k/v from their projections to the cache (forward.cc:395-459), see layer_kernels.hip:
// q <- rope(rms_norm(q, q_norm)) in place; cache K slot <- rope(rms_norm(k_raw, k_norm));
// cache V slot <- rms_norm(v_raw) (v_raw null: of k_raw). Token t is at position offset + t,
// slot (offset + t) % cap; when L > cap only the last cap tokens reach the cache.
struct AttnPrepareArgs {
    const uint32_t* pos = nullptr;   // non-null: the offset is read from *pos on the device
    const float2* rope_cs = nullptr; // non-null: (cos, sin) [positions][head_dim / 2] from
                                     // launch_rope_table, instead of computing them
    uint16_t* q;
    const uint16_t* k_raw;
    const uint16_t* v_raw;
    const uint16_t* q_norm;
    const uint16_t* k_norm;
    uint16_t* cache_k;
    uint16_t* cache_v;
    uint32_t L, n_heads, n_kv_heads, head_dim, rotated, offset, cap;
    float base, eps;
};
void launch_attn_prepare(const AttnPrepareArgs& a, hipStream_t stream);
// (cos, sin) of every position < positions and pair i < head_dim / 2, with rope_kernel's
// arithmetic (so a prepare that reads the table gives the bits of one that computes).
void launch_rope_table(float2* table, uint32_t positions, uint32_t head_dim, uint32_t rotated, float base,
                       hipStream_t stream);

// For each of m rows: residual <- bf16(residual + rms_norm(branch, w_post)); with scalar
// (device bf16 [1]) residual <- bf16(residual * scalar); with w_next, next <- rms_norm(
// residual, w_next). hidden a multiple of 64, at most residual_norm_max_hidden().
uint32_t residual_norm_max_hidden();
void launch_residual_norm(const uint16_t* branch, uint16_t* residual, const uint16_t* w_post, const uint16_t* scalar,
                          const uint16_t* w_next, uint16_t* next, uint32_t m, uint32_t hidden, float eps,
                          hipStream_t stream);

// The end of a replayed decode step: pos[0] += 1, ties[0] += sample->near_tie.
void launch_decode_advance(uint32_t* pos, uint32_t* ties, const HypTopKSample* sample, hipStream_t stream);

// mx.quantize(w, 64, 4, "affine") of bf16 [n, k].
void launch_q4_quantize(const uint16_t* w, uint32_t n, uint32_t k, uint32_t* wq,
                        uint16_t* scales, uint16_t* biases, hipStream_t stream);

// The same from the tiled resident layout (the embed table).
void launch_q4_dequantize_tiled(const Q4Matrix& w, const uint32_t* rows, uint32_t n_rows, float out_scale_bf16,
                                uint16_t* out, hipStream_t stream);

// mx.dequantize(..., bf16) of gathered rows; out_scale_bf16 != 0 multiplies each
// value by that bf16 constant with one more rounding.
void launch_q4_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                          uint32_t n_total, uint32_t k, const uint32_t* rows, uint32_t n_rows,
                          float out_scale_bf16, uint16_t* out, hipStream_t stream);

}  // namespace hyperion::hip
