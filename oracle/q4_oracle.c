/*
 * CPU oracle for the MLX-affine Q4/g64 path. TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, the smoke check and the benchmark's CPU-baseline leg as the checker,
 * never by the product library. Function-by-function provenance and pinning
 * status are in q4_oracle.h.
 *
 * Build flags matter: -ffp-contract=off (no fused multiply-add may be formed,
 * because every restated MLX op rounds on its own) and no -ffast-math.
 */
#include "q4_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define GROUP 64
#define NBINS 15.0f
#define EPS 1e-7f

/* Round-to-nearest-even fp32 -> bf16, quiet NaN kept quiet. MLX's bfloat16
 * conversion (mlx/types/bf16.h) does the same. */
uint16_t orc_bf16_from_f32(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return (uint16_t)((u >> 16) | 0x0040u);
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_f32_from_bf16(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_bf16_from_f32_array(const float* in, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_from_f32(in[i]);
}

void orc_f32_from_bf16_array(const uint16_t* in, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_from_bf16(in[i]);
}

static inline float bf(float f) { return orc_f32_from_bf16(orc_bf16_from_f32(f)); }

static inline float maxf_std(float a, float b) { return (a < b) ? b : a; } /* std::max */
static inline float minf_std(float a, float b) { return (b < a) ? b : a; } /* std::min */

/*
 * MLX affine quantize, one group of 64 (MLX 0.32.0 CPU backend; the reference
 * calls it at crates/hyperion-model/fixtures/build_gemma4_unified_tiny.py:54-57
 * and scripts/nax-probe.py:74-76):
 *   zero-point ("edge") rule - the scale is re-derived from the group's
 *   larger-magnitude extreme so that that extreme and zero are both exactly
 *   representable; all arithmetic in fp32 with IEEE division and rint.
 */
static void quantize_group(const uint16_t* w, uint32_t* wq, uint16_t* s_out, uint16_t* b_out) {
    float w_min = INFINITY;
    float w_max = -INFINITY;
    for (int j = 0; j < GROUP; ++j) {
        const float v = orc_f32_from_bf16(w[j]);
        w_max = maxf_std(w_max, v);
        w_min = minf_std(w_min, v);
    }
    const int mask = fabsf(w_min) > fabsf(w_max);
    float scale = maxf_std((w_max - w_min) / NBINS, EPS);
    scale = mask ? scale : -scale;
    const float edge = mask ? w_min : w_max;
    const float q0 = rintf(edge / scale);
    float bias = 0.0f;
    if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
    }
    for (int word = 0; word < GROUP / 8; ++word) {
        uint32_t packed = 0;
        for (int e = 0; e < 8; ++e) {
            float v = orc_f32_from_bf16(w[word * 8 + e]);
            v = rintf((v - bias) / scale);
            v = minf_std(maxf_std(v, 0.0f), NBINS);
            /* NaN input: both clamps keep NaN; define the code as 0. */
            const uint32_t code = (v == v) ? (uint32_t)v : 0u;
            packed |= code << (4 * e);
        }
        wq[word] = packed;
    }
    *s_out = orc_bf16_from_f32(scale);
    *b_out = orc_bf16_from_f32(bias);
}

void orc_quantize_q4g64(const uint16_t* w, int64_t n, int64_t k,
                        uint32_t* wq, uint16_t* scales, uint16_t* biases) {
    const int64_t groups = k / GROUP;
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t g = 0; g < groups; ++g) {
            quantize_group(w + r * k + g * GROUP, wq + r * (k / 8) + g * (GROUP / 8),
                           scales + r * groups + g, biases + r * groups + g);
        }
    }
}

/* Unpack code k of a row: word k/8, bits [4*(k%8), 4*(k%8)+4), low nibble first. */
static inline uint32_t code_at(const uint32_t* row, int64_t kk) {
    return (row[kk >> 3] >> (4 * (kk & 7))) & 0xFu;
}

/*
 * mx.dequantize(w, s, b, 64, 4, "affine", dtype=bf16) as used by ModelWeights::embed
 * (native/hyperion_mlx/src/weights_loader.cc:53-69) on gathered rows.
 */
void orc_dequantize_q4g64(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                          const uint32_t* rows, int64_t n_rows, int64_t k, int mode,
                          uint16_t* out) {
    const int64_t groups = k / GROUP;
    for (int64_t i = 0; i < n_rows; ++i) {
        const int64_t r = rows ? (int64_t)rows[i] : i;
        const uint32_t* wr = wq + r * (k / 8);
        for (int64_t kk = 0; kk < k; ++kk) {
            const float s = orc_f32_from_bf16(scales[r * groups + kk / GROUP]);
            const float b = orc_f32_from_bf16(biases[r * groups + kk / GROUP]);
            const float q = (float)code_at(wr, kk);
            float v;
            if (mode == 0) {
                v = bf(s * q);
                v = v + b;
            } else {
                v = s * q + b; /* s*q is exact in fp32: 8-bit x 4-bit significands */
            }
            out[i * k + kk] = orc_bf16_from_f32(v);
        }
    }
}

/* Ground truth, following the reference's own accuracy definition: dequantize and
 * multiply with no intermediate rounding (native/hyperion_mlx/tests/weights_test.cc:110-120). */
void orc_qmatmul_f64(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                     const uint16_t* biases, int64_t m, int64_t n, int64_t k, double* y) {
    const int64_t groups = k / GROUP;
    /* Each output is one thread's sequential sum: the result does not depend on the
     * thread count. */
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r) {
        const uint32_t* wr = wq + r * (k / 8);
        for (int64_t i = 0; i < m; ++i) {
            const uint16_t* xr = x + i * k;
            double acc = 0.0;
            for (int64_t g = 0; g < groups; ++g) {
                const double s = orc_f32_from_bf16(scales[r * groups + g]);
                const double b = orc_f32_from_bf16(biases[r * groups + g]);
                for (int64_t j = 0; j < GROUP; ++j) {
                    const int64_t kk = g * GROUP + j;
                    acc += (double)orc_f32_from_bf16(xr[kk]) * (s * (double)code_at(wr, kk) + b);
                }
            }
            y[i * n + r] = acc;
        }
    }
}

void orc_qmatmul_deq_f64(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                         const uint16_t* biases, int64_t m, int64_t n, int64_t k, int mode,
                         double* y) {
    /* Rows in parallel; each output is one thread's sequential sum (thread-count independent). */
#pragma omp parallel
    {
        double* row = (double*)malloc((size_t)k * sizeof(double));
        uint16_t* deq = (uint16_t*)malloc((size_t)k * sizeof(uint16_t));
        if (row == NULL || deq == NULL) abort();   /* a checker must not return partial output */
#pragma omp for schedule(static)
        for (int64_t r = 0; r < n; ++r) {
            const uint32_t id = (uint32_t)r;
            orc_dequantize_q4g64(wq, scales, biases, &id, 1, k, mode, deq);
            for (int64_t kk = 0; kk < k; ++kk) row[kk] = orc_f32_from_bf16(deq[kk]);
            for (int64_t i = 0; i < m; ++i) {
                const uint16_t* xr = x + i * k;
                double acc = 0.0;
                for (int64_t kk = 0; kk < k; ++kk) acc += (double)orc_f32_from_bf16(xr[kk]) * row[kk];
                y[i * n + r] = acc;
            }
        }
        free(row);
        free(deq);
    }
}

void orc_qmatmul_f32_grouped(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                             const uint16_t* biases, int64_t m, int64_t n, int64_t k, float* y) {
    const int64_t groups = k / GROUP;
    for (int64_t r = 0; r < n; ++r) {
        const uint32_t* wr = wq + r * (k / 8);
        for (int64_t i = 0; i < m; ++i) {
            const uint16_t* xr = x + i * k;
            float acc = 0.0f;
            for (int64_t g = 0; g < groups; ++g) {
                const float s = orc_f32_from_bf16(scales[r * groups + g]);
                const float b = orc_f32_from_bf16(biases[r * groups + g]);
                float sxq = 0.0f;
                float sx = 0.0f;
                for (int64_t j = 0; j < GROUP; ++j) {
                    const int64_t kk = g * GROUP + j;
                    const float xv = orc_f32_from_bf16(xr[kk]);
                    sxq += xv * (float)code_at(wr, kk);
                    sx += xv;
                }
                acc += s * sxq;
                acc += b * sx;
            }
            y[i * n + r] = acc;
        }
    }
}

/*
 * MLX CPU quantized_matmul with transpose=true, scalar loop, accumulator of the
 * input type: sum += x * (scale * q + bias), each op rounded to bf16 as MLX's
 * bfloat16_t operators do. Parity unpinned (see header).
 */
void orc_qmatmul_mlx_cpu_rows(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                              const uint16_t* biases, int64_t m, int64_t n0, int64_t n1,
                              int64_t k, uint16_t* y) {
    const int64_t groups = k / GROUP;
    const int64_t n_out = n1 - n0;
    for (int64_t i = 0; i < m; ++i) {
        const uint16_t* xr = x + i * k;
        for (int64_t r = n0; r < n1; ++r) {
            const uint32_t* wr = wq + r * (k / 8);
            float sum = 0.0f;
            for (int64_t g = 0; g < groups; ++g) {
                const float s = orc_f32_from_bf16(scales[r * groups + g]);
                const float b = orc_f32_from_bf16(biases[r * groups + g]);
                for (int64_t j = 0; j < GROUP; ++j) {
                    const int64_t kk = g * GROUP + j;
                    const float dq = bf(bf(s * (float)code_at(wr, kk)) + b);
                    sum = bf(sum + bf(orc_f32_from_bf16(xr[kk]) * dq));
                }
            }
            y[i * n_out + (r - n0)] = orc_bf16_from_f32(sum);
        }
    }
}

void orc_qmatmul_mlx_cpu(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                         const uint16_t* biases, int64_t m, int64_t n, int64_t k, uint16_t* y) {
    orc_qmatmul_mlx_cpu_rows(x, wq, scales, biases, m, 0, n, k, y);
}

/* The same loop with output rows dealt over `threads` OpenMP threads in blocks of 64
 * (each output row is still one sequential bf16 accumulation, so the result is
 * bit-identical to orc_qmatmul_mlx_cpu). */
void orc_qmatmul_mlx_cpu_mt(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                            const uint16_t* biases, int64_t m, int64_t n, int64_t k, int threads,
                            uint16_t* y) {
    const int64_t blocks = (n + 63) / 64;
    if (m == 1) {
#pragma omp parallel for schedule(static) num_threads(threads)
        for (int64_t bl = 0; bl < blocks; ++bl) {
            const int64_t r0 = bl * 64;
            const int64_t r1 = r0 + 64 < n ? r0 + 64 : n;
            orc_qmatmul_mlx_cpu_rows(x, wq, scales, biases, 1, r0, r1, k, y + r0);
        }
        return;
    }
    for (int64_t i = 0; i < m; ++i) orc_qmatmul_mlx_cpu_mt(x + i * k, wq, scales, biases, 1, n, k, threads, y + i * n);
}

/*
 * gelu_pytorch_tanh as the reference composes it (forward.cc:324-336): each MLX op
 * produces a bf16 array, constants are bf16 arrays.
 *   x3    = x * square(x)
 *   inner = bf16(0.044715) * x3 ; inner = inner + x ; inner = bf16(sqrt(2/pi)) * inner
 *   out   = (bf16(0.5) * x) * (bf16(1) + tanh(inner))
 */
static inline float gelu_chain(float xv) {
    const float c_coeff = bf(0.044715f);
    const float c_inner = bf(0.7978845608028654f);
    const float sq = bf(xv * xv);
    const float x3 = bf(xv * sq);
    float inner = bf(c_coeff * x3);
    inner = bf(inner + xv);
    inner = bf(c_inner * inner);
    const float t = bf(tanhf(inner));
    const float half_x = bf(0.5f * xv);
    const float one_t = bf(1.0f + t);
    return bf(half_x * one_t);
}

void orc_gelu_tanh_bf16(const uint16_t* x, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) {
        out[i] = orc_bf16_from_f32(gelu_chain(orc_f32_from_bf16(x[i])));
    }
}

/* ForwardPass::mlp (forward.cc:338-343): multiply(gelu_tanh(gate), up) in bf16. */
void orc_gelu_tanh_mul_bf16(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) {
        const float g = gelu_chain(orc_f32_from_bf16(gate[i]));
        out[i] = orc_bf16_from_f32(g * orc_f32_from_bf16(up[i]));
    }
}

/* ForwardPass::softcap (forward.cc:154-160): tanh(x / cap) * cap in the logits dtype. */
void orc_softcap_bf16(const uint16_t* x, int64_t n, float cap, uint16_t* out) {
    const float c = bf(cap);
    for (int64_t i = 0; i < n; ++i) {
        const float d = bf(orc_f32_from_bf16(x[i]) / c);
        const float t = bf(tanhf(d));
        out[i] = orc_bf16_from_f32(t * c);
    }
}

/* ForwardPass::embed scale (forward.cc:126-131): rows * bf16(sqrt(hidden)). */
void orc_scale_bf16(const uint16_t* x, int64_t n, float c, uint16_t* out) {
    const float cb = bf(c);
    for (int64_t i = 0; i < n; ++i) {
        out[i] = orc_bf16_from_f32(orc_f32_from_bf16(x[i]) * cb);
    }
}

/*
 * ForwardPass::sample_greedy (forward.cc:162-189): the row converted to fp32, then one
 * pass in index order keeping top1 (with its index) and top2; near_tie = top1 - top2 < 0.5.
 */
void orc_sample_greedy_bf16(const uint16_t* logits, int64_t n, uint32_t* token, float* logit,
                            int32_t* near_tie) {
    float top1 = -INFINITY;
    float top2 = -INFINITY;
    uint32_t arg = 0;
    for (int64_t i = 0; i < n; ++i) {
        const float v = orc_f32_from_bf16(logits[i]);
        if (v > top1) {
            top2 = top1;
            top1 = v;
            arg = (uint32_t)i;
        } else if (v > top2) {
            top2 = v;
        }
    }
    *token = arg;
    *logit = top1;
    *near_tie = (top1 - top2) < 0.5f ? 1 : 0;
}

/*
 * The top-k sidecar of the greedy epilogue (native/hyperion_mlx/src/model.cc:278-288): the
 * row converted to fp32, std::partial_sort of the indices by p[a] > p[b], the first
 * min(k, n) indices and their values. partial_sort leaves the order of equal values to the
 * library (and NaN breaks its comparator's ordering), so the order is defined here as:
 * larger value first (-0 == +0, as the comparator sees them), then the lower index; NaN
 * after every number, lower index first. Where the top k + 1 values are distinct numbers
 * this is partial_sort's result. Selection: k passes over the row, each taking the first
 * element in that order among those not yet taken. Returns the count; ids/values beyond
 * it are zero.
 */
static int topk_before(const float* p, int64_t a, int64_t b) {
    const int na = isnan(p[a]);
    const int nb = isnan(p[b]);
    if (na != nb) return nb;                /* a number before NaN */
    if (!na && p[a] != p[b]) return p[a] > p[b];
    return a < b;
}

uint32_t orc_sample_topk_bf16(const uint16_t* logits, int64_t n, uint32_t k, uint32_t* ids, float* values) {
    const uint32_t count = (int64_t)k < n ? k : (uint32_t)(n < 0 ? 0 : n);
    float* p = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    for (int64_t i = 0; i < n; ++i) p[i] = orc_f32_from_bf16(logits[i]);
    for (uint32_t j = 0; j < k; ++j) {
        ids[j] = 0;
        values[j] = 0.0f;
    }
    for (uint32_t j = 0; j < count; ++j) {
        int64_t best = -1;
        for (int64_t i = 0; i < n; ++i) {
            int taken = 0;
            for (uint32_t t = 0; t < j; ++t) taken |= (int64_t)ids[t] == i;
            if (taken) continue;
            if (best < 0 || topk_before(p, i, best)) best = i;
        }
        ids[j] = (uint32_t)best;
        values[j] = p[best];
    }
    free(p);
    return count;
}

/*
 * mx::fast::rms_norm(x, weight, eps) over rows (forward.cc:23-26) with the summation order
 * of the HIP kernels, so the two agree bit for bit:
 *   k a multiple of 64: per 64-element unit a sequential fp32 fma chain of squares; lane l
 *     of 64 adds units l, l + 64, ... in order; then an xor butterfly over the 64 lanes
 *     (offsets 32, 16, ..., 1; a + b == b + a, so every lane ends with the same total);
 *   otherwise: thread t of 256 runs an fma chain over elements t, t + 256, ...; a butterfly
 *     within each wave of 64; the four wave sums added in wave order.
 * inv = 1 / sqrtf(ss / k + eps); y = bf16(w * bf16(x * inv)), or bf16(x * inv) without w.
 */
static float butterfly64(float* v) {
    for (int off = 32; off > 0; off >>= 1) {
        float nv[64];
        for (int l = 0; l < 64; ++l) nv[l] = v[l] + v[l ^ off];
        for (int l = 0; l < 64; ++l) v[l] = nv[l];
    }
    return v[0];
}

/* ---- temperature sampling: ForwardPass::sample_stochastic (forward.cc:191-301) ----------
 *
 * The reference scales the fp32 logits by 1/temperature, takes the softmax, masks the tokens
 * outside the top-p nucleus (probability descending), below min_p times the largest
 * probability and outside the top-k (logit descending), then draws u from
 * uniform_real_distribution<float>(0, sz) and returns the first index whose running sum of
 * kept exp(t - max) reaches u (forward.cc:225-301). Its sort tie order and host summation
 * order are not fixed by its contract (hyperion_mlx.h:125-133: a statistical bar), so this
 * restates the defined algorithm of the HIP kernels, which fixes them:
 *   - 65536 bins over the bf16 value (bin 0 = largest, -0 as +0; -inf, +inf, NaN no bin);
 *     every filter keeps a prefix of (value descending, index ascending);
 *   - exp is st_exp below (the same fp32 operations as the device);
 *   - blocks of 64 bins; z = 16 wave sums in order, wave w adding in order the 64-lane xor
 *     butterflies of count * e over its blocks 16i + w; the mass before a bin = its block's
 *     start (the blocks' masses, each a Hillis-Steele scan over its bins, scanned in block
 *     order: within waves of 64 blocks plus the earlier waves' totals in order) + the scan of
 *     the block's masses before it;
 *   - the draw: chunks of 256 tokens, 4 per lane of a 64-lane wave; a lane's kept weights
 *     summed in token order, a Hillis-Steele scan over the lanes (the chunk total is its last
 *     lane), the chunk totals scanned the same way in groups of 64 chunks with the group
 *     totals added in order; the running sum at a token is chunk start + (lanes before + the
 *     lane's sum so far), and the token is the lowest index whose running sum reaches u;
 *   - rows whose scaled logits hold +inf or NaN draw the last index, rows with no finite
 *     scaled logit (and none of those) draw index 0 - what the reference's arithmetic gives.
 * canon is the uniform in [0, 1) (std::generate_canonical<float> of std::mt19937_64 seeded
 * with the request's RNG state; u = sz * canon). */
#define ST_BINS 65536u
#define ST_NOBIN ST_BINS
#define ST_THREADS 1024u
#define ST_PER 64u
#define ST_NONE 0xFFFFFFFFu

static uint32_t st_bin_of(uint16_t h) {
    uint32_t b = h;
    if (b == 0x8000u) b = 0u;
    if ((b & 0x7F80u) == 0x7F80u) return ST_NOBIN;
    const uint32_t ok = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
    return 0xFFFFu - ok;
}

static float st_bin_value(uint32_t d) {
    const uint32_t ok = 0xFFFFu - d;
    const uint32_t b = (ok & 0x8000u) ? (ok & 0x7FFFu) : (~ok & 0xFFFFu);
    return orc_f32_from_bf16((uint16_t)b);
}

/* exp(x), x <= 0: Cody-Waite reduction by ln 2 (ln 2 split as 0.693145751953125 +
 * 1.42860677e-06), the degree-7 Taylor polynomial of exp on |r| <= 0.35 in Horner form,
 * times 2^k; 0 at or below -86 (results stay normal numbers). Unfused fp32 operations. */
float orc_det_exp(float x) {
    if (!(x > -86.0f)) return 0.0f;
    const float kf = rintf(x * 1.44269502f);
    const float r = (x - kf * 0.693145751953125f) - kf * 1.42860677e-06f;
    float p = 1.98412701e-04f;
    p = p * r + 1.38888892e-03f;
    p = p * r + 8.33333377e-03f;
    p = p * r + 4.16666679e-02f;
    p = p * r + 1.66666672e-01f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    const int k = (int)kf;
    uint32_t e = (uint32_t)(k + 127) << 23;
    float scale;
    memcpy(&scale, &e, 4);
    return p * scale;
}

static float st_weight(uint32_t d, float inv_temp, float max_t) {
    return orc_det_exp(st_bin_value(d) * inv_temp - max_t);
}

/* Inclusive Hillis-Steele scan of 64 lanes: in step d (1, 2, 4, ..., 32) lane l >= d adds the
 * value lane l - d held before the step. */
static void st_hs_scan64(float* v) {
    for (uint32_t d = 1u; d < 64u; d <<= 1) {
        float t[64];
        for (uint32_t l = 0; l < 64u; ++l) t[l] = l >= d ? v[l] + v[l - d] : v[l];
        memcpy(v, t, sizeof(t));
    }
}

/* Exclusive prefix over the 1024 threads' values: the scan within each wave of 64, plus the
 * earlier waves' totals added in order; a[ST_THREADS] = the total. */
static void st_prefix_f(float* a) {
    float off = 0.0f;
    for (uint32_t w = 0; w < ST_THREADS / 64u; ++w) {
        float v[64];
        memcpy(v, a + 64u * w, sizeof(v));
        st_hs_scan64(v);
        for (uint32_t l = 0; l < 64u; ++l) a[64u * w + l] = off + (l != 0u ? v[l - 1u] : 0.0f);
        off = off + v[63];
    }
    a[ST_THREADS] = off;
}

static void st_prefix_u(uint32_t* a) {
    uint32_t run = 0u;
    for (uint32_t j = 0; j < ST_THREADS; ++j) {
        const uint32_t v = a[j];
        a[j] = run;
        run = run + v;
    }
    a[ST_THREADS] = run;
}

void orc_sample_stochastic_bf16(const uint16_t* logits, uint32_t vocab, float inv_temp, float top_p, float min_p,
                                int32_t top_k, float canon, uint32_t* token, float* logit, uint32_t* kept) {
    uint32_t* cnt = (uint32_t*)calloc(ST_BINS, sizeof(uint32_t));
    int inf_nan = 0, neg_inf = 0;
    for (uint32_t i = 0; i < vocab; ++i) {
        const uint32_t d = st_bin_of(logits[i]);
        if (d < ST_BINS) cnt[d] += 1u;
        else if (logits[i] == 0xFF80u) neg_inf = 1;
        else inf_nan = 1;
    }
    uint32_t top = ST_NOBIN;
    for (uint32_t d = 0; d < ST_BINS && top == ST_NOBIN; ++d) {
        if (cnt[d] != 0u) top = d;
    }
    const float max_t = top != ST_NOBIN ? st_bin_value(top) * inv_temp : 0.0f;
    int mode = 0;   /* 0 kept, 1 index 0, 2 the last index */
    if (inf_nan || (neg_inf && inv_temp == 0.0f) || isnan(inv_temp) || isnan(max_t) || max_t == INFINITY) {
        mode = 2;
    } else if (top == ST_NOBIN || max_t == -INFINITY) {
        mode = 1;
    }
    if (mode != 0 || vocab == 0u) {
        const uint32_t arg = mode == 2 && vocab != 0u ? vocab - 1u : 0u;
        *token = arg;
        *logit = vocab != 0u ? orc_f32_from_bf16(logits[arg]) : -INFINITY;
        if (kept) *kept = 0u;
        free(cnt);
        return;
    }

    /* Blocks of 64 bins (block b = bins 64b .. 64b + 63); wave w of 16 takes blocks 16i + w.
     * z: per block a butterfly over its bins of count * e, each wave adding its blocks in
     * order i = 0..63, the 16 wave sums in order. */
#define ST_BLOCKS (ST_BINS / 64u)
    float z = 0.0f;
    for (uint32_t w = 0; w < ST_THREADS / 64u; ++w) {
        float zw = 0.0f;
        for (uint32_t i = 0; i < ST_BLOCKS / 16u; ++i) {
            const uint32_t b = 16u * i + w;
            float lanes[64];
            for (uint32_t l = 0; l < 64u; ++l) {
                const uint32_t d = 64u * b + l;
                lanes[l] = cnt[d] != 0u ? (float)cnt[d] * st_weight(d, inv_temp, max_t) : 0.0f;
            }
            zw = zw + butterfly64(lanes);
        }
        z = z + zw;
    }

    /* Probability mass per bin, c * (e / z); per block a Hillis-Steele scan over its bins
     * (the block's mass is the last lane's), then the masses and token counts before each
     * block in block order (st_prefix_f: waves of 64 blocks, offsets added in order). */
    float* mass = (float*)malloc(sizeof(float) * ST_BINS);
    float bm[ST_BLOCKS + 1];
    uint32_t bc[ST_BLOCKS + 1];
    for (uint32_t b = 0; b < ST_BLOCKS; ++b) {
        float v[64];
        uint32_t t = 0u;
        for (uint32_t l = 0; l < 64u; ++l) {
            const uint32_t d = 64u * b + l;
            mass[d] = cnt[d] != 0u ? (float)cnt[d] * (st_weight(d, inv_temp, max_t) / z) : 0.0f;
            v[l] = mass[d];
            t += cnt[d];
        }
        st_hs_scan64(v);
        bm[b] = v[63];
        bc[b] = t;
    }
    st_prefix_f(bm);
    st_prefix_u(bc);
    const uint32_t total = bc[ST_BLOCKS];

    /* top-p: per non-empty bin, the running mass before it (block start + the scan of the
     * block's masses before it); where that plus count * p reaches top_p, the smallest count
     * t that does by bisection; the lowest position over bins. */
    uint32_t np = total;
    if (top_p > 0.0f && top_p <= 1.0f) {
        uint32_t best = ST_NONE;
        for (uint32_t b = 0; b < ST_BLOCKS; ++b) {
            float v[64];
            for (uint32_t l = 0; l < 64u; ++l) v[l] = mass[64u * b + l];
            st_hs_scan64(v);
            uint32_t seen = bc[b];
            for (uint32_t l = 0; l < 64u; ++l) {
                const uint32_t d = 64u * b + l;
                const uint32_t c = cnt[d];
                const float cb = bm[b] + (l != 0u ? v[l - 1u] : 0.0f);
                if (c != 0u) {
                    const float p = st_weight(d, inv_temp, max_t) / z;
                    if (cb + (float)c * p >= top_p) {
                        uint32_t lo = 1u, hi = c;
                        while (lo < hi) {
                            const uint32_t mid = (lo + hi) >> 1;
                            if (cb + (float)mid * p >= top_p) hi = mid; else lo = mid + 1u;
                        }
                        if (seen + lo < best) best = seen + lo;
                    }
                }
                seen += c;
            }
        }
        if (best != ST_NONE) np = best;
    }
    free(mass);
#undef ST_BLOCKS
    /* min-p: the tokens whose probability is at least min_p * (1 / z). */
    uint32_t nm = total;
    if (min_p > 0.0f && min_p < 1.0f) {
        const float thr = min_p * (1.0f / z);
        nm = 0u;
        for (uint32_t d = 0; d < ST_BINS; ++d) {
            if (cnt[d] != 0u && st_weight(d, inv_temp, max_t) / z >= thr) nm += cnt[d];
        }
    }
    const uint32_t nk = top_k > 0 && (uint32_t)top_k < vocab ? (uint32_t)top_k : total;
    uint32_t n = np < nm ? np : nm;
    if (nk < n) n = nk;
    if (total < n) n = total;
    uint32_t cut_bin = 0u, cut_count = 0u, seen = 0u;
    for (uint32_t d = 0; d < ST_BINS; ++d) {
        if (seen + cnt[d] >= n && cnt[d] != 0u) {
            cut_bin = d;
            cut_count = n - seen;
            break;
        }
        seen += cnt[d];
    }
    free(cnt);
    if (kept) *kept = n;

    /* The draw over chunks of 256 tokens (lane l of a chunk: its tokens 4l..4l+3). kept(i):
     * bin < cut_bin, or the cut bin within its first cut_count tokens in index order. */
#define ST_CHUNK 256u
    const uint32_t chunks = (vocab + ST_CHUNK - 1u) / ST_CHUNK;
    const uint32_t groups = (chunks + 63u) / 64u;
    float* wt = (float*)malloc(sizeof(float) * (size_t)chunks * ST_CHUNK);   /* kept weight or -1 */
    uint32_t cut_seen = 0u;
    for (uint32_t i = 0; i < chunks * ST_CHUNK; ++i) {
        wt[i] = -1.0f;
        if (i >= vocab) continue;
        const uint32_t d = st_bin_of(logits[i]);
        const int keep = d < cut_bin || (d == cut_bin && cut_seen < cut_count);
        if (d == cut_bin) cut_seen += 1u;
        if (keep) wt[i] = orc_det_exp(orc_f32_from_bf16(logits[i]) * inv_temp - max_t);
    }
    float* before = (float*)malloc(sizeof(float) * (size_t)chunks * 64u);   /* lane sums before */
    float* start = (float*)calloc((size_t)groups * 64u, sizeof(float));
    for (uint32_t c = 0; c < chunks; ++c) {
        float v[64];
        for (uint32_t l = 0; l < 64u; ++l) {
            float sum = 0.0f;
            for (uint32_t k = 0; k < 4u; ++k) {
                const float w = wt[c * ST_CHUNK + 4u * l + k];
                if (w >= 0.0f) sum = sum + w;
            }
            v[l] = sum;
        }
        st_hs_scan64(v);
        for (uint32_t l = 0; l < 64u; ++l) before[c * 64u + l] = l != 0u ? v[l - 1u] : 0.0f;
        start[c] = v[63];   /* the chunk total, replaced by its start below */
    }
    float run = 0.0f;
    for (uint32_t g = 0; g < groups; ++g) {
        float v[64];
        memcpy(v, start + 64u * g, sizeof(v));   /* chunks past the row hold 0 */
        st_hs_scan64(v);
        for (uint32_t l = 0; l < 64u; ++l) start[64u * g + l] = run + (l != 0u ? v[l - 1u] : 0.0f);
        run = run + v[63];
    }
    const float sz = run;
    const float u = sz * canon + 0.0f;
    uint32_t arg = ST_NONE;
    if (u <= 0.0f) {
        arg = 0u;
    } else {
        for (uint32_t i = 0; i < vocab && arg == ST_NONE; ++i) {
            const float w = wt[i];
            if (w < 0.0f) continue;
            const uint32_t c = i / ST_CHUNK, l = (i % ST_CHUNK) / 4u;
            float part = 0.0f;
            for (uint32_t j = c * ST_CHUNK + 4u * l; j <= i; ++j)
                if (wt[j] >= 0.0f) part = part + wt[j];
            if (u <= start[c] + (before[c * 64u + l] + part)) arg = i;
        }
    }
#undef ST_CHUNK
    free(wt);
    free(before);
    free(start);
    if (arg >= vocab) arg = vocab - 1u;
    *token = arg;
    *logit = orc_f32_from_bf16(logits[arg]);
}

void orc_rms_norm_bf16(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t k, float eps, uint16_t* y) {
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* xr = x + r * k;
        uint16_t* yr = y + r * k;
        float ss;
        if (k % 64 == 0) {
            const int64_t units = k / 64;
            float lanes[64];
            for (int l = 0; l < 64; ++l) {
                float acc = 0.0f;
                for (int64_t u = l; u < units; u += 64) {
                    float us = 0.0f;
                    for (int64_t e = 0; e < 64; ++e) {
                        const float v = orc_f32_from_bf16(xr[u * 64 + e]);
                        us = fmaf(v, v, us);
                    }
                    acc += us;
                }
                lanes[l] = acc;
            }
            ss = butterfly64(lanes);
        } else {
            float waves[4];
            for (int wv = 0; wv < 4; ++wv) {
                float lanes[64];
                for (int l = 0; l < 64; ++l) {
                    float acc = 0.0f;
                    for (int64_t i = wv * 64 + l; i < k; i += 256) {
                        const float v = orc_f32_from_bf16(xr[i]);
                        acc = fmaf(v, v, acc);
                    }
                    lanes[l] = acc;
                }
                waves[wv] = butterfly64(lanes);
            }
            ss = 0.0f;
            for (int wv = 0; wv < 4; ++wv) ss += waves[wv];
        }
        const float inv = 1.0f / sqrtf(ss / (float)k + eps);
        for (int64_t i = 0; i < k; ++i) {
            float v = bf(orc_f32_from_bf16(xr[i]) * inv);
            if (w != NULL) v = orc_f32_from_bf16(w[i]) * v;
            yr[i] = orc_bf16_from_f32(v);
        }
    }
}

/*
 * mx::fast::rope(x, dims = head_dim, traditional = false, base | freqs, scale = 1, offset)
 * (rope.cc:16-75) on x [rows, heads, head_dim] bf16, row r at position offset + r. Pairs
 * (i, i + head_dim/2) for i < head_dim/2 rotate by theta = fp32(pos) * inv_freq_i, with
 * inv_freq_i = fp32(base^(-2i/head_dim)) for i < rotated/2 and 0 above (the proportional
 * scheme's infinite frequencies: identity). Both are computed in double and rounded to
 * fp32 once; cos and sin likewise from the fp32 theta. Then, in fp32 without fusion,
 *   y_i = bf16(x_i c - x_{i+D/2} s),  y_{i+D/2} = bf16(x_i s + x_{i+D/2} c).
 */
void orc_rope_bf16(const uint16_t* x, int64_t rows, int64_t heads, int64_t head_dim, int64_t rotated,
                   double base, int64_t offset, uint16_t* y) {
    const int64_t half = head_dim / 2;
    for (int64_t r = 0; r < rows; ++r) {
        const float pos = (float)(offset + r);
        for (int64_t i = 0; i < half; ++i) {
            const float inv = (2 * i < rotated) ? (float)pow(base, -2.0 * (double)i / (double)head_dim) : 0.0f;
            const float theta = pos * inv;
            const float c = (float)cos((double)theta);
            const float sn = (float)sin((double)theta);
            for (int64_t h = 0; h < heads; ++h) {
                const int64_t b = (r * heads + h) * head_dim;
                const float x1 = orc_f32_from_bf16(x[b + i]);
                const float x2 = orc_f32_from_bf16(x[b + i + half]);
                const float a1 = x1 * c;
                const float a2 = x2 * sn;
                const float b1 = x1 * sn;
                const float b2 = x2 * c;
                y[b + i] = orc_bf16_from_f32(a1 - a2);
                y[b + i + half] = orc_bf16_from_f32(b1 + b2);
            }
        }
    }
}

/*
 * mx::fast::scaled_dot_product_attention as ForwardPass::attention calls it
 * (native/hyperion_mlx/src/forward.cc:376-508): scale 1.0 (Gemma 4 drops 1/sqrt(d)), a
 * boolean mask from absolute positions (build_mask, forward.cc:345-373: key k is visible to
 * query q when k <= q, and for a sliding layer also k > q - window), grouped-query heads
 * (query head h reads kv head h / (n_heads / n_kv_heads)). In fp64 on the bf16 inputs.
 * Keys are the cache's prefix positions [offset - prefix_len, offset) (slot = pos % cap)
 * followed by the chunk's L positions [offset, offset + L). q [L][n_heads][d], k and v
 * [L][n_kv][d], cache_k and cache_v [cap][n_kv][d]; out [L][n_heads][d].
 */
void orc_attention_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* cache_k,
                       const uint16_t* cache_v, int64_t cap, int64_t L, int64_t n_heads, int64_t n_kv,
                       int64_t d, int64_t offset, int64_t prefix_len, int64_t window, double* out) {
    const int64_t group = n_heads / n_kv;
    const int64_t T = prefix_len + L;
#pragma omp parallel
    {
        double* s = (double*)malloc((size_t)(T > 0 ? T : 1) * sizeof(double));
#pragma omp for schedule(dynamic, 4)
        for (int64_t th = 0; th < L * n_heads; ++th) {
            const int64_t t = th / n_heads;
            const int64_t h = th - t * n_heads;
            const int64_t qpos = offset + t;
            const int64_t hk = h / group;
            const uint16_t* qv = q + (t * n_heads + h) * d;
            double m = -INFINITY;
            for (int64_t j = 0; j < T; ++j) {
                const int64_t kpos = offset - prefix_len + j;
                const int visible = kpos <= qpos && (window == 0 || kpos > qpos - window);
                if (!visible) {
                    s[j] = -INFINITY;
                    continue;
                }
                const uint16_t* kv = j < prefix_len ? cache_k + ((kpos % cap) * n_kv + hk) * d
                                                    : k + ((kpos - offset) * n_kv + hk) * d;
                double acc = 0.0;
                for (int64_t e = 0; e < d; ++e) acc += (double)orc_f32_from_bf16(qv[e]) * (double)orc_f32_from_bf16(kv[e]);
                s[j] = acc;
                if (acc > m) m = acc;
            }
            double sum = 0.0;
            for (int64_t j = 0; j < T; ++j) {
                s[j] = s[j] == -INFINITY ? 0.0 : exp(s[j] - m);
                sum += s[j];
            }
            double* o = out + (t * n_heads + h) * d;
            for (int64_t e = 0; e < d; ++e) o[e] = 0.0;
            for (int64_t j = 0; j < T; ++j) {
                if (s[j] == 0.0) continue;
                const int64_t kpos = offset - prefix_len + j;
                const uint16_t* vv = j < prefix_len ? cache_v + ((kpos % cap) * n_kv + hk) * d
                                                    : v + ((kpos - offset) * n_kv + hk) * d;
                const double w = s[j] / sum;
                for (int64_t e = 0; e < d; ++e) o[e] += w * (double)orc_f32_from_bf16(vv[e]);
            }
        }
        free(s);
    }
}
