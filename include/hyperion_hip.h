/*
 * hyperion_hip.h - C ABI of the MI355X (gfx950) Q4/g64 quantized-linear engine.
 *
 * Drop-in for the reference's quantized-linear path: every quantized linear in the
 * reference is mlx::core::quantized_matmul(x, w, scales, biases, transpose=true,
 * 64, 4, "affine") (native/hyperion_mlx/src/weights.h:26-37). This library replaces
 * that call, the tied LM head (forward.cc:137-152), the MLP gating (forward.cc:324-343),
 * the embed dequantize-gather (weights_loader.cc:53-69), the quantize used to make
 * weights (mx.quantize, build_gemma4_unified_tiny.py:54-57) and the weight residency
 * built by load_model_weights (weights_loader.cc:71-153).
 *
 * Conventions follow the reference ABI (native/hyperion_mlx/include/hyperion_mlx.h):
 *  - every function returns HypStatus (same values as hyperion_mlx.h:12-21);
 *  - a non-OK return stores a message in a thread-local buffer read by
 *    hyp_last_error (abi_error.cc:7-19); an OK return clears it;
 *  - no C++ exception crosses the boundary (the abi_call pattern, runtime.mm:79-97);
 *  - handles are opaque and magic-tagged; create(out) rejects a NULL out pointer;
 *    free(&h) sets h to NULL, is a no-op on NULL and rejects a wrong magic
 *    (model.cc:170-207);
 *  - input buffers are borrowed for the call only;
 *  - one thread drives a device's work; calls are synchronous with respect to the
 *    host only where stated (kernels are enqueued on the caller's stream).
 *
 * Layouts (MLX affine, transpose=true; tensor shapes as stored by mlx-lm):
 *  - packed weight  uint32 [n, k/8]: code of column c lives in word c/8, bits
 *                   [4*(c%8), 4*(c%8)+4) (lowest k in the lowest nibble);
 *  - scales, biases bf16 [n, k/64];  dequant(W)[r, c] = scale[r, c/64] * q + bias[r, c/64];
 *  - activations    bf16 row-major x [m, k], y [m, n]; y = x * dequant(W)^T.
 * bf16 values cross the ABI as their 16-bit patterns (uint16_t or void*).
 * "device pointer" means memory from hyp_device_alloc (or any hipMalloc'd memory
 * on the current device).
 */
#ifndef HYPERION_HIP_H
#define HYPERION_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HYP_HIP_ABI_VERSION 1u

/* Same numbering as the reference (hyperion_mlx.h:12-21). OOM_GOVERNOR is unused here:
 * device allocation failures report HYP_STATUS_INTERNAL as the reference does for
 * allocation outside governor admission (model.cc:442-452). */
typedef enum HypStatus {
    HYP_STATUS_OK = 0,
    HYP_STATUS_INVALID_ARGUMENT = 1,
    HYP_STATUS_NOT_FOUND = 2,
    HYP_STATUS_IO = 3,
    HYP_STATUS_OOM_GOVERNOR = 4,
    HYP_STATUS_UNSUPPORTED = 5,
    HYP_STATUS_INTERNAL = 6,
    HYP_STATUS_CANCELLED = 7
} HypStatus;

/* Opaque handles. */
typedef struct HypQWeightOpaque* HypQWeight;   /* magic "HPQW": one resident Q4 projection */
typedef struct HypQModelOpaque* HypQModel;     /* magic "HPQM": all resident Q4 projections */
typedef struct HypStreamOpaque* HypStream;     /* a HIP stream (hipStream_t) */
typedef struct HypEventOpaque* HypEvent;       /* a HIP event (hipEvent_t) */
typedef struct HypGraphOpaque* HypGraph;       /* magic "HPGR": an instantiated HIP graph */

/* Device and build facts; replaces the Apple platform canary (runtime.mm:223-284). */
typedef struct HypRuntimeInfo {
    uint32_t abi_version;
    int32_t device_count;
    int32_t device;                 /* current device */
    uint32_t compute_units;
    uint64_t hbm_bytes;
    uint32_t clock_khz;
    uint32_t l2_bytes;
    char arch_name[64];             /* e.g. "gfx950:sramecc+:xnack-" */
    char device_name[128];
} HypRuntimeInfo;

/* Projection selector for hyp_qmodel_linear (weights_loader.cc:132-141 names). */
typedef enum HypProj {
    HYP_PROJ_Q = 0,
    HYP_PROJ_K = 1,
    HYP_PROJ_V = 2,
    HYP_PROJ_O = 3,
    HYP_PROJ_GATE = 4,
    HYP_PROJ_UP = 5,
    HYP_PROJ_DOWN = 6
} HypProj;

/* Epilogue applied by hyp_qmatmul_ex to the bf16 output. */
typedef enum HypEpilogue {
    HYP_EPILOGUE_NONE = 0,
    HYP_EPILOGUE_SOFTCAP = 1        /* y = bf16(bf16(tanh(bf16(y / cap))) * cap), forward.cc:154-160 */
} HypEpilogue;

/* ForwardPass::GreedySample (forward.h:104-108); near_tie is a bool there. */
typedef struct HypGreedySample {
    uint32_t token_id;              /* argmax token */
    float logit;                    /* the winning logit (bf16 value as fp32) */
    uint32_t near_tie;              /* 1 when top1 - top2 < 0.5, else 0 */
} HypGreedySample;

/* The top-k sidecar's size, HYP_TOP_K_LOGPROBS (hyperion_mlx.h:145). */
#define HYP_TOP_K_LOGPROBS 8

/* ForwardPass::StochasticSample (forward.h:125-131) as the greedy epilogue fills it
 * (model.cc:272-288), with GreedySample's near_tie (forward.h:104-108): the greedy token
 * and logit, and the top_k_count = min(HYP_TOP_K_LOGPROBS, vocab) largest post-softcap
 * logits (fp32 of the bf16 values; the reference calls them logprobs) with their ids,
 * descending. Entries past top_k_count are zero. 80 bytes. */
typedef struct HypTopKSample {
    uint32_t token_id;
    float logit;
    uint32_t near_tie;
    uint32_t top_k_count;
    uint32_t top_k_ids[HYP_TOP_K_LOGPROBS];
    float top_k_logprobs[HYP_TOP_K_LOGPROBS];
} HypTopKSample;

/* ---- errors and runtime ------------------------------------------------------- */

/* Copy the calling thread's last error into buffer (NUL-terminated, truncated).
 * Replaces hyp_last_error (hyperion_mlx.h:41, runtime.mm:286-298). */
HypStatus hyp_last_error(char* buffer, size_t buffer_len);

/* Fill *out with the ABI version and the current device's facts.
 * Replaces hyp_runtime_canary (hyperion_mlx.h:38). UNSUPPORTED when no HIP device. */
HypStatus hyp_runtime_info(HypRuntimeInfo* out);

/* Device memory, streams and events. The reference gets these from MLX
 * (lazy arrays moved to the GPU on first use, weights_loader.h:70-79, and explicit
 * mx::Stream arguments, weights.h:26); a C caller of this engine gets them here. */
HypStatus hyp_device_alloc(size_t bytes, void** out_ptr);
HypStatus hyp_device_free(void** ptr);
/* A non-blocking HIP stream plus a 306 KiB device workspace for the calls that need one
 * (hyp_sample_greedy, hyp_sample_greedy_topk, hyp_sample_stochastic). destroy waits for the
 * device before freeing the workspace. */
HypStatus hyp_stream_create(HypStream* out_stream);
HypStatus hyp_stream_destroy(HypStream* stream);
HypStatus hyp_stream_synchronize(HypStream stream);
/* Copies are enqueued on stream and complete before hyp_stream_synchronize returns.
 * Host buffers may be pageable (then the copy is synchronous with the host). */
HypStatus hyp_memcpy_htod(void* dst_device, const void* src_host, size_t bytes, HypStream stream);
HypStatus hyp_memcpy_dtoh(void* dst_host, const void* src_device, size_t bytes, HypStream stream);
HypStatus hyp_memcpy_dtod(void* dst_device, const void* src_device, size_t bytes, HypStream stream);
HypStatus hyp_memset_device(void* dst_device, int value, size_t bytes, HypStream stream);
HypStatus hyp_event_create(HypEvent* out_event);
HypStatus hyp_event_destroy(HypEvent* event);
HypStatus hyp_event_record(HypEvent event, HypStream stream);
/* Milliseconds between two recorded events; waits for `end` to complete. */
HypStatus hyp_event_elapsed_ms(HypEvent start, HypEvent end, float* out_ms);

/* Graph capture of a launch sequence (e.g. one decode step) so it replays without
 * per-launch host work; the reference has no counterpart (MLX evaluates its lazy graph
 * at mx::eval, forward.cc:171). Between begin and end, hyp_qmatmul, hyp_qmatmul_ex,
 * hyp_qmatmul_group, hyp_qmlp_gate_up_gelu and hyp_qmatmul_group_rmsnorm with m <= 4, hyp_rms_normalize, hyp_quantize_q4g64,
 * hyp_dequantize_q4g64, hyp_embed, hyp_sample_greedy, hyp_sample_greedy_topk, hyp_kv_cache_write,
 * hyp_attention, hyp_rope and the copies on `stream` are
 * recorded instead of run (they allocate nothing). Calls that may allocate or clear
 * memory - the matmul entries on their GEMM path (m > 4) and hyp_memset_device - check
 * the stream and return INVALID_ARGUMENT while it is capturing, before enqueueing
 * anything; the capture stays open and usable. The recorded pointers and handles must
 * stay valid while the graph is used. */
HypStatus hyp_graph_capture_begin(HypStream stream);
HypStatus hyp_graph_capture_end(HypStream stream, HypGraph* out_graph);
/* Enqueue one replay of the graph on stream. */
HypStatus hyp_graph_launch(HypGraph graph, HypStream stream);
HypStatus hyp_graph_free(HypGraph* graph);

/* ---- resident Q4 weights (QuantizedLinear, weights.h:18-25; make_proj,
 *      weights_loader.cc:33-45) --------------------------------------------------- */

/* Copy one projection from host memory into device-resident storage.
 * w: uint32 [n, k/8]; scales/biases: bf16 [n, k/64] (MLX affine layout).
 * group_size != 64 or bits != 4 -> UNSUPPORTED (the locked quantization,
 * model.cc:73-74, hyperion-model/src/weights.rs:35-58); n == 0, k == 0 or
 * k % 64 != 0 -> INVALID_ARGUMENT. */
HypStatus hyp_qweight_create(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                             uint32_t n, uint32_t k, uint32_t group_size, uint32_t bits,
                             HypQWeight* out_weight);
/* Same, from device pointers (copied; the caller keeps ownership of its buffers). */
HypStatus hyp_qweight_create_device(const uint32_t* w, const void* scales, const void* biases,
                                    uint32_t n, uint32_t k, uint32_t group_size, uint32_t bits,
                                    HypStream stream, HypQWeight* out_weight);
HypStatus hyp_qweight_free(HypQWeight* weight);
HypStatus hyp_qweight_shape(HypQWeight weight, uint32_t* out_n, uint32_t* out_k);
/* Copy the resident projection back to host in MLX layout (synchronous). */
HypStatus hyp_qweight_export(HypQWeight weight, uint32_t* w, uint16_t* scales, uint16_t* biases);

/* ---- quantized matmul ---------------------------------------------------------- */

/* y[m, n] = x[m, k] * dequant(W)^T with fp32 accumulation, bf16 out.
 * Replaces QuantizedLinear::apply (weights.h:26-37) for every M: m <= 4 runs the
 * weight-streaming decode kernel, larger m the tiled GEMM (both on bf16 MFMA).
 * x and y are device pointers; m == 0 is a no-op. */
HypStatus hyp_qmatmul(HypQWeight weight, const void* x, uint32_t m, void* y, HypStream stream);

/* hyp_qmatmul that allocates nothing: no hipMalloc, hipMallocAsync, hipFree or other
 * allocating call, on any path. It has no counterpart in the reference; it is for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation). The kernels and k splits are those of hyp_qmatmul, so the output
 * is the same bits; where hyp_qmatmul's prefill GEMM (m > 4) splits k, the fp32 partial
 * sums go to a fixed 64 MiB device scratch array that the library holds on each device
 * it runs on until the process ends (enough for every projection of a 12B layer at
 * m <= 2048). A call whose partials would exceed it returns INVALID_ARGUMENT and runs
 * nothing. All calls on one device share that scratch: calls that overlap on one device
 * (e.g. on two streams without ordering between them) race; calls on one stream are
 * ordered and safe. Nothing in the scratch needs clearing between calls. */
HypStatus hyp_qmatmul_noalloc(HypQWeight weight, const void* x, uint32_t m, void* y, HypStream stream);

/* hyp_qmatmul with an epilogue; HYP_EPILOGUE_SOFTCAP with cap > 0 is the tied
 * LM head + softcap of ForwardPass::lm_head/softcap (forward.cc:137-160). */
HypStatus hyp_qmatmul_ex(HypQWeight weight, const void* x, uint32_t m, void* y,
                         HypEpilogue epilogue, float cap, HypStream stream);

/* ys[i][m, n_i] = x[m, k] * dequant(W_i)^T for count (1..HYP_QMATMUL_GROUP_MAX) weights
 * that share k: the q/k/v projections of one attention block, which the reference applies
 * to the same normed input one after another (forward.cc:395,399,409). At m <= 4 this is
 * one launch over all of their rows; larger m runs the GEMM per weight. Same results as
 * count separate hyp_qmatmul calls. */
#define HYP_QMATMUL_GROUP_MAX 3u
HypStatus hyp_qmatmul_group(const HypQWeight* weights, uint32_t count, const void* x, uint32_t m,
                            void* const* ys, HypStream stream);

/* hyp_rms_normalize(x, norm_weight, m, k, eps) followed by hyp_qmatmul_group on its
 * output, with the same results bit for bit: the pre-attention input_layernorm and q/k/v
 * of one block (forward.cc:521, 395-409). norm_weight is the norm's bf16 weight [k]
 * (device, 16-byte aligned) or NULL for the weightless form. At m <= 4 it is one launch
 * that normalises the rows in on-chip memory and does not write them back; x is left
 * unchanged either way. */
HypStatus hyp_qmatmul_group_rmsnorm(const HypQWeight* weights, uint32_t count, const void* x,
                                    const void* norm_weight, uint32_t m, float eps, void* const* ys,
                                    HypStream stream);

/* h[m, n] = gelu_tanh(x * dequant(G)^T) * (x * dequant(U)^T), the gate/up half of
 * ForwardPass::mlp (forward.cc:338-343) with gelu_tanh rounded op-by-op in bf16 as
 * forward.cc:324-336 composes it. gate and up must share (n, k). */
HypStatus hyp_qmlp_gate_up_gelu(HypQWeight gate, HypQWeight up, const void* x, uint32_t m,
                                void* h, HypStream stream);

/* ---- quantize / dequantize ----------------------------------------------------- */

/* mx.quantize(w, group_size=64, bits=4, mode="affine") of a bf16 [n, k] device matrix
 * into w_out uint32 [n, k/8], scales_out/biases_out bf16 [n, k/64] (device). w and w_out
 * must be 16-byte aligned (INVALID_ARGUMENT otherwise; device allocations are). */
HypStatus hyp_quantize_q4g64(const void* w, uint32_t n, uint32_t k, uint32_t* w_out,
                             void* scales_out, void* biases_out, HypStream stream);

/* mx.dequantize(..., dtype=bfloat16) of rows rows[0..n_rows) (rows == NULL: rows
 * 0..n_rows) of a Q4 matrix of k columns into out bf16 [n_rows, k]; each value is
 * bf16(scale*q + bias), one rounding as MLX's dequantize (weights_loader.cc:60-69; the
 * reference's 12B embed golden, forward_12b_test.cc:218, fits only this rounding).
 * If out_scale != 0 the result is further multiplied
 * by bf16(out_scale) and rounded (the embed scale, forward.cc:126-131). Row ids
 * are device uint32; the kernel never reads outside the table: an id >= n_total
 * yields a row of zeros (mx::take would raise; ids are not visible to the host
 * without a synchronizing copy, so the check happens on the device). */
HypStatus hyp_dequantize_q4g64(const uint32_t* w, const void* scales, const void* biases,
                               uint32_t n_total, uint32_t k, const uint32_t* rows,
                               uint32_t n_rows, float out_scale, void* out, HypStream stream);

/* ModelWeights::embed + ForwardPass::embed (weights_loader.cc:53-69, forward.cc:126-131):
 * gather rows ids[0..n_ids) of the resident table, dequantize to bf16 and multiply
 * by bf16(sqrt(k)). ids are device uint32 < n (out-of-range ids produce zero rows). */
HypStatus hyp_embed(HypQWeight table, const uint32_t* ids, uint32_t n_ids, void* out,
                    HypStream stream);

/* mx::fast::rms_norm(x, weight, eps) over rows (forward.cc:23-26): for each of m rows of
 * k bf16 values, y[r] = bf16(w * bf16(x[r] / sqrt(mean(x[r]^2) + eps))) with fp32
 * statistics, w the bf16 weight [k] (device, 16-byte aligned when k % 64 == 0); weight ==
 * NULL is the parameterless form, y[r] = bf16(x[r] / sqrt(...)). The reference applies the
 * weighted form as input_layernorm, post_attention_layernorm and the feed-forward norms
 * (forward.cc:521-529) and per head as q_norm and k_norm (rows = tokens x heads, k =
 * head_dim, forward.cc:400-405), and the weightless one as v_norm (forward.cc:403-412).
 * y may alias x. eps must be finite and >= 0. */
HypStatus hyp_rms_normalize(const void* x, const void* weight, uint32_t m, uint32_t k, float eps, void* y,
                            HypStream stream);

/* mx::fast::rope(x, dims = head_dim, traditional = false, base | freqs, scale = 1, offset)
 * as Rope::apply does it (rope.cc:16-75) on x [rows, heads, head_dim] bf16 (device), row r
 * at position offset + r; y may alias x. Pair (i, i + head_dim/2) of every head rotates by
 * theta = fp32(offset + r) * fp32(base^(-2i / head_dim)) when i < rotated_dims/2, and is
 * copied otherwise: the local layers' default scheme is rotated_dims = head_dim (256,
 * base 1e4), the global layers' proportional scheme rotated_dims = 128 of head_dim 512
 * (base 1e6; its frequencies are base^(2i / head_dim) over the full head_dim, rope.cc:16-33).
 * inv_freq, cos and sin are computed in double and rounded to fp32; the rotation is fp32
 * (no fused multiply-add), rounded to bf16. offset + rows must stay below 2^24. */
HypStatus hyp_rope(const void* x, uint32_t rows, uint32_t heads, uint32_t head_dim, uint32_t rotated_dims, float base,
                   uint32_t offset, void* y, HypStream stream);

/* ForwardPass::sample_greedy (forward.cc:162-189) on the device, replacing its host copy
 * of the logits and the CPU scan: for each of `rows` rows of `vocab` bf16 logits
 * (row-major, device memory), out[r] (device memory) receives the first index of the
 * largest value, that value, and whether it leads the largest other value by less than
 * 0.5. NaN logits are skipped; a row with no value above -inf (or vocab == 0) gives
 * token 0. The reference samples the last position: pass logits + (m - 1) * vocab and
 * rows = 1 after the softcap LM head (hyp_qmatmul_ex). Uses a 48 KiB device workspace
 * owned by the stream (made by hyp_stream_create): a graph captured on a stream keeps
 * using that stream's workspace, so replay it on that stream (or one whose work is
 * ordered with it) and only while the stream exists. */
HypStatus hyp_sample_greedy(const void* logits, uint32_t rows, uint32_t vocab, HypGreedySample* out,
                            HypStream stream);

/* The greedy epilogue with its top-k sidecar (model.cc:272-288) on the device, replacing
 * the host copy of the row and the std::partial_sort there: out[r] (device memory) gets
 * hyp_sample_greedy's token, logit and near_tie for row r, and its HYP_TOP_K_LOGPROBS
 * largest values with their ids. partial_sort leaves the order of equal values to the
 * library, so it is defined here: larger value first (-0 and +0 equal), then the lower
 * index; NaN after every number, lower index first. Where the largest
 * HYP_TOP_K_LOGPROBS + 1 values are distinct this is exactly partial_sort's result.
 * vocab is at most 2^23 (INVALID_ARGUMENT above). Same workspace and capture rules as
 * hyp_sample_greedy. */
HypStatus hyp_sample_greedy_topk(const void* logits, uint32_t rows, uint32_t vocab, HypTopKSample* out,
                                 HypStream stream);

/* ---- attention and the KV caches (forward.cc:376-508, kv_cache.h:33,143) ------------- */

/* One layer's KV cache on the device: K and V [capacity][num_kv_heads][head_dim] bf16, token
 * position p in slot p % capacity. A sliding layer's ring (LocalKvCache) is a cache of at
 * least its window; a global layer's cache (GlobalKvCache) is given the context length as
 * capacity - the reference grows it in 256-token steps, which 288 GB of HBM does not need.
 * The handle also owns the workspace of decode attention's split keys (fixed size), so
 * attention on a capturing stream allocates nothing. head_dim: 64, 128, 256 or 512. */
typedef struct HypKvCacheOpaque* HypKvCache;   /* magic "HPKV" */
HypStatus hyp_kv_cache_create(uint32_t capacity, uint32_t num_kv_heads, uint32_t head_dim, HypKvCache* out_cache);
HypStatus hyp_kv_cache_free(HypKvCache* cache);
/* Device pointers of the cache's K and V tensors (valid until free). */
HypStatus hyp_kv_cache_buffers(HypKvCache cache, void** out_k, void** out_v);
/* Write n_tokens of k/v [n_tokens][num_kv_heads][head_dim] (device, bf16) at positions
 * pos0 .. pos0 + n_tokens - 1 (LocalKvCache::append_committed, GlobalKvCache::append);
 * when n_tokens > capacity only the last capacity tokens are written (the earlier ones would
 * be overwritten in the ring). */
HypStatus hyp_kv_cache_write(HypKvCache cache, const void* k, const void* v, uint32_t n_tokens, uint32_t pos0,
                             HypStream stream);
/* mx::fast::scaled_dot_product_attention as ForwardPass::attention calls it: scale 1.0,
 * the boolean mask of build_mask (forward.cc:345-373: key position p visible to the query
 * at position offset + t when p <= offset + t and, with window > 0, p > offset + t -
 * window), grouped-query heads (query head h reads kv head h / (n_heads / num_kv_heads)).
 * q [L][n_heads][head_dim], the chunk's k/v [L][num_kv_heads][head_dim] (post-norm, k
 * post-rope), out [L][n_heads][head_dim], all device bf16, 16-byte aligned. The keys are
 * the cache's positions [offset - prefix_len, offset) followed by the chunk's L positions
 * [offset, offset + L): call it before hyp_kv_cache_write of the chunk, so a ring's prefix
 * is read before the chunk overwrites its slots. prefix_len <= offset and <= capacity (a
 * sliding layer passes min(window, offset), a global one offset). fp32 scores and softmax,
 * P rounded to bf16 for the P.V products, output rounded to bf16. */
HypStatus hyp_attention(const void* q, const void* k, const void* v, uint32_t L, uint32_t n_heads, HypKvCache cache,
                        uint32_t offset, uint32_t prefix_len, uint32_t window, void* out, HypStream stream);

/* ---- the rest of a decoder layer (forward.cc:395-459, 518-539) ---------------------- */

/* From the q/k/v projections to the cache append, one launch (forward.cc:400-459): for
 * token t of the chunk (position offset + t, cache slot (offset + t) % capacity),
 *   q[t][h]        <- rope(rms_norm(q[t][h], q_norm))            in place, every head h;
 *   cache K[slot]  <- rope(rms_norm(k_raw[t][j], k_norm))        every kv head j;
 *   cache V[slot]  <- rms_norm(v_raw[t][j]) without a weight     (v_norm; v_raw NULL reads
 *                                                                 k_raw: the K = V layers).
 * q [L][n_heads][head_dim], k_raw / v_raw [L][num_kv_heads][head_dim], q_norm / k_norm bf16
 * [head_dim], all device memory, 16-byte aligned; rope as hyp_rope with rotated_dims and
 * rope_base. The bits are those of hyp_rms_normalize, hyp_rope and hyp_kv_cache_write in
 * sequence. Then hyp_attention(q, NULL, NULL, L, ...) reads the chunk from the cache, which
 * needs prefix_len + L <= capacity. */
HypStatus hyp_attention_prepare(void* q, const void* k_raw, const void* v_raw, uint32_t L, uint32_t n_heads,
                                HypKvCache cache, const void* q_norm, const void* k_norm, float eps,
                                uint32_t rotated_dims, float rope_base, uint32_t offset, HypStream stream);

/* The Gemma sandwich closing a block (ForwardPass::decoder_layer, forward.cc:518-539), one
 * launch over m rows of hidden bf16 (device, 16-byte aligned):
 *   residual <- bf16(residual + rms_norm(branch, post_weight));
 *   residual <- bf16(residual * scalar[0])          when scalar (device bf16 [1]) is non-NULL
 *                                                   (the layer_scalar after the MLP half);
 *   next     <- rms_norm(residual, next_weight)     when next_weight is non-NULL (the next
 *                                                   block's input norm; next [m][hidden]).
 * Each norm has the bits of hyp_rms_normalize. hidden: a multiple of 64, at most 16384. */
HypStatus hyp_residual_rms_norm(const void* branch, void* residual, const void* post_weight, const void* scalar,
                                const void* next_weight, void* next, uint32_t m, uint32_t hidden, float eps,
                                HypStream stream);

/* ---- the model, its KV state and the step ABI (hyperion_mlx.h:50-248) -------------------
 * The reference's model-level entry points over this library's kernels: hyp_model_load
 * makes the projections, norm vectors and layer scalars resident; hyp_prefill_chunk and
 * hyp_decode_block run embed -> layers -> final norm -> softcap LM head -> greedy sample
 * on the device (ForwardPass::forward, forward.cc:543-563; model.cc:515-740). The types
 * below have the reference's names and layouts. Each call is synchronous and runs on the
 * model's own HIP stream; one thread drives a model and its states. Differences: no
 * governor (governor_state is always READY and peak/active bytes are 0; every cache is
 * allocated at its final size by hyp_kvstate_create, so there is nothing to admit),
 * token ids >= vocab_size are rejected, and the temperature draw fixes the orders the
 * reference leaves to its library (hyp_sample_stochastic). */
typedef struct HypModelOpaque* HypModel;             /* magic "HPMD" */
typedef struct HypKvStateOpaque* HypKvState;         /* magic "HPKS" */
typedef struct HypStepResultOpaque* HypStepResult;   /* magic "HPSR" */

typedef enum HypTextModelType { HYP_GEMMA4_TEXT = 0, HYP_GEMMA4_UNIFIED_TEXT = 1 } HypTextModelType;
typedef enum HypLayerType { HYP_LAYER_SLIDING = 0, HYP_LAYER_FULL = 1 } HypLayerType;
typedef enum HypGovernorState {
    HYP_GOVERNOR_READY = 0,
    HYP_GOVERNOR_SOFT_PAUSED = 1,
    HYP_GOVERNOR_HARD_REJECT = 2
} HypGovernorState;

/* hyperion_mlx.h:75-80. */
typedef struct HypRopeSpec {
    double theta;
    int has_partial_rotary_factor;
    float partial_rotary_factor;
    int proportional;
} HypRopeSpec;

typedef struct HypMoeConfig {
    uint32_t num_experts;
    uint32_t top_k;
    uint32_t moe_intermediate_size;
} HypMoeConfig;

/* hyperion_mlx.h:89-116, validated as Geometry::validate does (geometry.cc:78-130). */
typedef struct HypGeometryParams {
    HypTextModelType model_type;
    uint32_t hidden_size;
    uint32_t intermediate_size;
    uint32_t num_hidden_layers;
    const HypLayerType* layer_types;
    uint32_t num_attention_heads;
    uint32_t head_dim_local;
    uint32_t head_dim_global;
    uint32_t num_kv_heads_local;
    uint32_t num_kv_heads_global;
    int attention_k_eq_v_global;
    uint32_t num_kv_shared_layers;
    uint32_t sliding_window;
    HypRopeSpec rope_local;
    HypRopeSpec rope_global;
    float final_logit_softcapping;
    float rms_norm_eps;
    int attention_bias;
    uint32_t vocab_size;
    uint32_t max_position_embeddings;
    int tie_word_embeddings;
    uint32_t ple_hidden_per_layer_input;
    uint32_t ple_vocab_per_layer_input;
    int use_double_wide_mlp;
    int has_moe;
    HypMoeConfig moe;
} HypGeometryParams;

/* hyperion_mlx.h:119-123. */
typedef struct HypTokenStream {
    const uint32_t* tokens;
    uint32_t count;
    int is_prompt;
} HypTokenStream;

/* hyperion_mlx.h:134-140. */
typedef struct HypSamplingConfig {
    float temperature;
    int32_t top_k;
    float top_p;
    float min_p;
    uint64_t seed;
} HypSamplingConfig;

/* hyperion_mlx.h:157-176. */
typedef struct {
    uint32_t token_id;
    float logit;
    uint64_t peak_mlx_bytes;
    uint64_t active_mlx_bytes;
    uint64_t phys_footprint_bytes;
    uint64_t local_kv_bytes;
    uint64_t global_kv_bytes;
    float local_kv_eval_ms;
    float global_kv_eval_ms;
    HypGovernorState governor_state;
    uint32_t near_tie_events;
    uint32_t top_k_logprob_count;
    uint32_t top_k_logprob_ids[HYP_TOP_K_LOGPROBS];
    float top_k_logprob_values[HYP_TOP_K_LOGPROBS];
} HypStepResultFields;

HypStatus hyp_model_create(HypModel* out_model);
HypStatus hyp_model_free(HypModel* model);
/* Load the artifact in weights_path (the hyp_qmodel_load rules, plus the norm vectors
 * input_layernorm, post_attention_layernorm, pre_feedforward_layernorm,
 * post_feedforward_layernorm, self_attn.q_norm, self_attn.k_norm, layer_scalar and the
 * final language_model.model.norm) for `geometry`, on the current device. A loaded model
 * rejects a second load; a missing directory is NOT_FOUND. */
HypStatus hyp_model_load(HypModel model, const HypGeometryParams* geometry, const char* weights_path);
/* One LocalKvCache ring of sliding_window + 2048 positions per sliding layer and one
 * GlobalKvCache of max_position_embeddings positions per global layer (kv.cc). */
HypStatus hyp_kvstate_create(HypModel model, HypKvState* out_kvstate);
/* Frees the state; valid after a step returned HYP_STATUS_INTERNAL (hyperion_mlx.h:192-194). */
HypStatus hyp_kvstate_free(HypKvState* kvstate);
/* Prefill a fresh state with tokens->count tokens in 2048-token chunks; the result holds
 * the greedy token after the last one (top_k_logprob_count 0). A state consumed by a failed
 * decode returns HYP_STATUS_INTERNAL until it is freed (hyperion_mlx.h:196-198). A failed
 * prefill leaves the state reusable: the next prefill rewrites every position it reads. */
HypStatus hyp_prefill_chunk(HypModel model, HypKvState kvstate, const HypTokenStream* tokens,
                            HypStepResult out_result);
/* n_tokens greedy steps from the state's last token; the result holds the last step's
 * token and the number of steps whose top-2 gap was < 0.5. A decode that fails after its
 * first step is enqueued consumes the state: it and every later prefill or decode on that
 * state return HYP_STATUS_INTERNAL until it is freed and recreated (hyperion_mlx.h:204-208,
 * DirectKvExecutionGuard model.cc:79-105). */
HypStatus hyp_decode_block(HypModel model, HypKvState kvstate, uint32_t n_tokens, HypStepResult out_result);
/* The same with a sampling config (hyperion_mlx.h:210-231, model.cc:743-960): NULL or
 * temperature 0 is the greedy path plus the top-k sidecar (near_tie_events 0, as
 * model.cc:262-288 reports it); a malformed config is INVALID_ARGUMENT (model.cc:234-257);
 * temperature > 0 draws each token as hyp_sample_stochastic does, on the device, with the
 * top-k sidecar of the pre-filter logits. The prefill draws with the RNG state config->seed
 * (model.cc:841); a decode block starts every call from config->seed and advances the state
 * per step as state * 6364136223846793005 + 1442695040888963407 (model.cc:926-944), so the
 * same seed and prompt give the same tokens. */
HypStatus hyp_prefill_chunk_sampled(HypModel model, HypKvState kvstate, const HypTokenStream* tokens,
                                    const HypSamplingConfig* config, HypStepResult out_result);
HypStatus hyp_decode_block_sampled(HypModel model, HypKvState kvstate, uint32_t n_tokens,
                                   const HypSamplingConfig* config, HypStepResult out_result);

/* ForwardPass::sample_stochastic (forward.cc:191-322) of one row of vocab bf16 logits
 * (device memory) into *out (device memory, 80 bytes), replacing the host copy of the row,
 * the host softmax, sorts and draw: config (host memory) is validated as
 * validate_sampling_config does (model.cc:234-257; INVALID_ARGUMENT); NULL or temperature 0
 * gives hyp_sample_greedy_topk's result. Otherwise t = logit * (1/temperature), the softmax
 * of t, the top-p nucleus, min-p and top-k filters (each as the reference applies it) and a
 * draw u = sz * U, where U = std::generate_canonical<float, 24> of std::mt19937_64 seeded with
 * rng_state (what std::uniform_real_distribution<float>(0, sz) draws under libstdc++) and sz
 * the kept total: the first index whose running sum of the kept exp(t - max t) reaches u;
 * token_id, logit (its pre-filter value), near_tie 0, and the top-k sidecar of the
 * pre-filter logits. The reference leaves the order of equal probabilities and of its fp32
 * sums to its library (a statistical bar, hyperion_mlx.h:125-133); here they are fixed:
 * equal values are kept lowest index first, and the sums run in the kernels' fixed order,
 * so the result is a deterministic function of (logits, config, rng_state). A +inf or NaN
 * scaled logit makes the reference's draw total NaN and its draw the last index; so here.
 * With no finite scaled logit (and no such value) it draws index 0, as the reference's zero
 * total does. vocab is at most 2^23. Uses the stream's workspace (hyp_sample_greedy's
 * capture rules; a captured call keeps its rng_state). */
HypStatus hyp_sample_stochastic(const void* logits, uint32_t vocab, const HypSamplingConfig* config,
                                uint64_t rng_state, HypTopKSample* out, HypStream stream);
HypStatus hyp_step_result_create(HypStepResult* out_result);
HypStatus hyp_step_result_free(HypStepResult* result);
HypStatus hyp_step_result_fields(HypStepResult result, HypStepResultFields* out_fields);
/* Device memory of a model and one of its KV states, counted in the formats this library
 * keeps resident: the quantization-aware replacement of the governor's weight estimate
 * (peak_within_budget, governor.cc:601-640), which counts every weight at 2 bytes (bf16) and
 * so puts the Q4/g64 12B at 24.7 GB instead of the 6.6 GB that is resident. */
typedef struct HypMemoryReport {
    uint64_t weight_bytes;              /* the Q4/g64 projections and the tied embedding / LM head
                                         * in the tiled resident layout (0.5625 B per weight,
                                         * plus padding to 16 rows and 128 columns) */
    uint64_t norm_bytes;                /* norm vectors, layer scalars, the final norm (bf16) */
    uint64_t kv_local_bytes;            /* one state's sliding-layer rings, K and V */
    uint64_t kv_global_bytes;           /* one state's global-layer caches, K and V */
    uint64_t state_bytes;               /* one state's sampled token and device counters */
    uint64_t scratch_bytes;             /* the model's activation buffers for a 2048-token chunk,
                                         * attention and sampling workspaces, RoPE tables */
    uint64_t dense_bf16_weight_bytes;   /* the same projections at 2 bytes per weight */
} HypMemoryReport;
/* What hyp_model_load and one hyp_kvstate_create allocate for `geometry` (host only: no
 * artifact, no device). */
HypStatus hyp_geometry_memory(const HypGeometryParams* geometry, HypMemoryReport* out);
/* The loaded model's allocations, summed buffer by buffer, with one state's KV as
 * hyp_kvstate_create allocates it. */
HypStatus hyp_model_memory(HypModel model, HypMemoryReport* out);

/* ForwardPass::embed + forward (forward.cc:126-131, 543-563) as forward_test.cc drives it:
 * `count` host token ids at positions offset .. offset + count - 1, their K/V appended to
 * the state's caches, and the final-normalised hidden rows copied to hidden_out (host, bf16
 * [count][hidden_size]). The state's cursor does not move. */
HypStatus hyp_model_forward_hidden(HypModel model, HypKvState kvstate, const uint32_t* ids, uint32_t count,
                                   uint32_t offset, uint16_t* hidden_out);

/* ---- decode-step program (the per-token layer loop, forward.cc:558-563, run by
 *      hyp_decode_block, model.cc:703-718) ------------------------------------------ */

/* An ordered list of decode-size (m <= 4) quantized-linear ops run by ONE launch: a
 * persistent kernel with one 16-wave workgroup per compute unit walks the ops, and op i
 * starts only when every workgroup has finished op i - 1 (device-memory arrival counters).
 * It replaces the per-op launches of a decode step, each of which carries a fixed cost of
 * several microseconds; the next op's weights stream in while its input is awaited.
 * Op i may read anything an earlier op wrote and overwrite anything an earlier op read.
 * Each op gives the same bits as its per-call entry point:
 *   HYP_STEP_QMATMUL          count 1..3 weights sharing k: hyp_qmatmul / hyp_qmatmul_group
 *   HYP_STEP_QMATMUL_RMSNORM  the same on rms-normalised x rows: hyp_qmatmul_group_rmsnorm
 *   HYP_STEP_GATE_UP_GELU     weights[0] gate, weights[1] up, output y[0]:
 *                             hyp_qmlp_gate_up_gelu */
typedef struct HypStepProgramOpaque* HypStepProgram;   /* magic "HPSP" */

typedef enum HypStepOpKind {
    HYP_STEP_QMATMUL = 0,
    HYP_STEP_QMATMUL_RMSNORM = 1,
    HYP_STEP_GATE_UP_GELU = 2
} HypStepOpKind;

typedef struct HypStepOp {
    uint32_t kind;                  /* HypStepOpKind */
    uint32_t count;                 /* weights used: 1..3, or 2 for GATE_UP_GELU */
    HypQWeight weights[3];
    const void* x;                  /* device bf16 [m, k] */
    void* y[3];                     /* device bf16 [m, n_i] (GATE_UP_GELU: y[0] only) */
    float eps;                      /* QMATMUL_RMSNORM */
    uint32_t reserved;              /* 0 */
    const void* norm_weight;        /* QMATMUL_RMSNORM: the norm's bf16 weight [k], or NULL */
} HypStepOp;

/* Validate the ops for m rows (1..4) and keep a device copy of them. The weights and
 * buffers are borrowed: they must stay valid while the program is used. An op whose k
 * needs more than one register-resident range per wave (k > 16384, or k > 4096 for
 * GATE_UP_GELU), or whose x rows exceed the LDS, is UNSUPPORTED. spin_limit bounds how
 * long a workgroup polls for the others at an op boundary (0: the default, about 2 s);
 * a run that exceeds it gives up, leaving its outputs undefined, and the next
 * hyp_step_program_check reports it. */
HypStatus hyp_step_program_create(const HypStepOp* ops, uint32_t n_ops, uint32_t m, uint32_t spin_limit,
                                  HypStepProgram* out_program);
/* Enqueue one run on stream (one cooperative launch; not recordable into a graph: the
 * call returns INVALID_ARGUMENT while the stream is capturing). Runs of one program must
 * be ordered (one stream). */
HypStatus hyp_step_program_run(HypStepProgram program, HypStream stream);
/* Wait for the device; INTERNAL if a run since the last check gave up waiting (the
 * program is then reset and can run again), else OK. */
HypStatus hyp_step_program_check(HypStepProgram program);
HypStatus hyp_step_program_free(HypStepProgram* program);

/* ---- weight residency (load_model_weights, weights_loader.cc:71-153) ------------ */

/* Load every *.safetensors shard in dir, resolve the MLX names
 * language_model.model.layers.{i}.{self_attn.{q,k,v,o}_proj | mlp.{gate,up,down}_proj}
 * .{weight,scales,biases} and language_model.model.embed_tokens.* and make each a
 * resident HypQWeight. A layer without v_proj is a global (K = V) layer.
 * num_layers == 0 means "as many as the shards hold". Missing dir -> NOT_FOUND;
 * unreadable shard -> IO; malformed header or a missing tensor -> INVALID_ARGUMENT. */
HypStatus hyp_qmodel_load(const char* dir, uint32_t num_layers, HypQModel* out_model);
HypStatus hyp_qmodel_free(HypQModel* model);
HypStatus hyp_qmodel_num_layers(HypQModel model, uint32_t* out_num_layers);
/* Borrowed handle (owned by the model; do not free). A global layer's V -> NOT_FOUND. */
HypStatus hyp_qmodel_linear(HypQModel model, uint32_t layer, HypProj proj, HypQWeight* out_weight);
HypStatus hyp_qmodel_embed(HypQModel model, HypQWeight* out_weight);

#ifdef __cplusplus
}
#endif

#endif
