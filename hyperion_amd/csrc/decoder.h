// The decoder around the Q4 projections, device-resident: the model-level half of the
// reference's native engine re-expressed on HIP buffers and the kernels of this library.
//
//   Geometry::from_abi / validate   native/hyperion_mlx/src/geometry.cc:23-130
//   Decoder (ForwardPass)           forward.cc:95-135 (construction, embed, final_norm),
//                                   :376-508 (attention), :509-541 (decoder_layer),
//                                   :543-563 (forward), :137-189 (lm_head, softcap, greedy)
//   DecoderState (KvState)          kv_cache.h:33 (LocalKvCache), :143 (GlobalKvCache)
//   prefill / decode_block          model.cc:515-627 (hyp_prefill_chunk), :629-740
//                                   (hyp_decode_block), :262-301 (the greedy sidecar)
//
// Differences of form, not of results:
//  * every KV cache is allocated once at its final size. A sliding layer's ring holds
//    window + kChunkTokens positions, so a chunk is appended before its attention and the
//    window it needs is never overwritten; a global layer's cache holds
//    max_position_embeddings positions (the reference grows it in 256-token steps; HBM holds
//    the 12B's 8 global caches at 262144 positions in 4.3 GB).
//  * the sampled token stays in device memory between decode steps: the next step's embed
//    gather reads it there, so a decode block makes one host round trip, at its end.
//  * a decode step is one HIP graph, captured once per state and replayed per token: the
//    position lives in device memory (the kernels that depend on it read it there and a
//    last node advances it), so a replay needs no host work beyond its launch.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "hyperion_hip.h"
#include "qlinear.h"

namespace hyperion::model {

// Prefill chunk size (model.cc:574, kPrefillChunkSize).
constexpr uint32_t kChunkTokens = 2048;

struct RopeParams {
    double theta = 0.0;
    bool has_partial = false;
    float partial = 0.0f;
    bool proportional = false;
};

struct Geometry {
    uint32_t hidden = 0;
    uint32_t intermediate = 0;
    std::vector<LayerType> types;
    uint32_t heads = 0;
    uint32_t head_dim_local = 0;
    uint32_t head_dim_global = 0;
    uint32_t kv_heads_local = 0;
    uint32_t kv_heads_global = 0;
    bool k_eq_v_global = true;
    uint32_t window = 0;
    RopeParams rope_local;
    RopeParams rope_global;
    float softcap = 0.0f;
    float eps = 0.0f;
    uint32_t vocab = 0;
    uint32_t max_positions = 0;

    // Geometry::from_abi + validate (geometry.cc:23-130): INVALID_ARGUMENT for what the
    // reference rejects, UNSUPPORTED for the variants this build does not run (MoE,
    // per-layer inputs, double-wide MLP, shared KV layers, attention bias, head dims other
    // than 64/128/256/512, sizes not a multiple of 64).
    static Geometry from_abi(const HypGeometryParams& p);

    [[nodiscard]] uint32_t num_layers() const noexcept { return static_cast<uint32_t>(types.size()); }
    // Rope::Rope (rope.cc:36-56): the proportional scheme rotates floor(prf * head_dim)
    // rounded down to even dims; the default scheme the whole head.
    [[nodiscard]] uint32_t rotated_dims(LayerType kind) const noexcept;
};

// HypMemoryReport's fields (the planned or the allocated device bytes).
struct MemoryReport {
    uint64_t weight_bytes = 0;
    uint64_t norm_bytes = 0;
    uint64_t kv_local_bytes = 0;
    uint64_t kv_global_bytes = 0;
    uint64_t state_bytes = 0;
    uint64_t scratch_bytes = 0;
    uint64_t dense_bf16_weight_bytes = 0;
};

// What a Decoder and one DecoderState allocate for `g`, from the geometry alone.
MemoryReport plan_memory(const Geometry& g);

struct LayerCache {
    DeviceBuffer k;   // [cap][kv_heads][head_dim] bf16
    DeviceBuffer v;
    uint32_t cap = 0;
    uint32_t kv_heads = 0;
    uint32_t head_dim = 0;
};

// An instantiated HIP graph, destroyed with its owner.
class GraphExec {
  public:
    GraphExec() = default;
    explicit GraphExec(hipGraphExec_t exec) : exec_(exec) {}
    ~GraphExec();
    GraphExec(const GraphExec&) = delete;
    GraphExec& operator=(const GraphExec&) = delete;
    GraphExec(GraphExec&& o) noexcept : exec_(o.exec_) { o.exec_ = nullptr; }
    GraphExec& operator=(GraphExec&& o) noexcept;
    [[nodiscard]] hipGraphExec_t get() const noexcept { return exec_; }

  private:
    hipGraphExec_t exec_ = nullptr;
};

// One sequence's KV state (KvState, kv.h) plus its autoregressive cursor (model.cc:606-607).
struct DecoderState {
    std::vector<LayerCache> caches;   // one per layer, in layer order
    uint32_t offset = 0;              // tokens committed
    uint32_t last_token = 0;
    DeviceBuffer cur;                 // HypTopKSample: the last sampled token, on the device
    DeviceBuffer counters;            // uint32 [2]: the device-side position and near-tie count
    GraphExec step;                   // one decode step, captured at the first decode
    GraphExec sampled_step;           // the same with the temperature draw, at the first sampled decode
    uint64_t local_bytes = 0;
    uint64_t global_bytes = 0;
    // Set when a decode failed after its first replay was enqueued: the KV rows, the device
    // cursor and the sampled token may have moved past `offset`, so the state is consumed and
    // every later step on it is refused until it is freed (model.cc:79-105, :155).
    bool consumed = false;
};

// One sampled step as the ABI reports it.
struct StepSample {
    HypTopKSample sample{};
    uint32_t near_tie_events = 0;
};

class Decoder {
  public:
    Decoder(Geometry geometry, ModelWeights weights);
    ~Decoder();
    Decoder(const Decoder&) = delete;
    Decoder& operator=(const Decoder&) = delete;

    [[nodiscard]] const Geometry& geometry() const noexcept { return geo_; }
    [[nodiscard]] hipStream_t stream() const noexcept { return stream_; }

    // build_kv_state (kv.cc) at final sizes.
    [[nodiscard]] DecoderState make_state() const;

    // ForwardPass::embed + forward over `count` tokens at positions offset.. (host ids),
    // appending their K/V; the final-normalised hidden rows [count][hidden] bf16 are copied
    // to the host. Does not move the cursor. Synchronous.
    void forward_hidden(DecoderState& st, const uint32_t* ids, uint32_t count, uint32_t offset,
                        uint16_t* hidden_out);
    // hyp_prefill_chunk: chunked prefill of a fresh state, then the epilogue on the last
    // position. With `sampling` (a validated config with temperature > 0:
    // hyp_prefill_chunk_sampled) the token is drawn with the config's seed (model.cc:841).
    // Synchronous.
    StepSample prefill(DecoderState& st, const uint32_t* ids, uint32_t count,
                       const HypSamplingConfig* sampling = nullptr);
    // hyp_decode_block: n_tokens greedy steps from the cursor; with `sampling`
    // (hyp_decode_block_sampled) each step draws, the RNG state starting from the config's
    // seed and advancing per step (model.cc:924-944). Synchronous.
    StepSample decode(DecoderState& st, uint32_t n_tokens, const HypSamplingConfig* sampling = nullptr);
    // The allocated buffers, summed (KV and state as make_state allocates them).
    [[nodiscard]] MemoryReport memory() const;

  private:
    // embed + all layers over L <= kChunkTokens tokens whose ids are in device memory.
    // final_rows: all L final-normalised rows there; otherwise the last row into last_.
    // d_pos non-null (a replayable step): the position is read from *d_pos on the device
    // and `offset` is unused.
    void forward_chunk(DecoderState& st, const uint32_t* d_ids, uint32_t L, uint32_t offset, uint16_t* final_rows,
                       const uint32_t* d_pos = nullptr);
    // lm_head + softcap + greedy with the top-k sidecar of last_ into *d_out; with `draw`
    // the temperature draw (the parameters in stoch_ws_) then replaces the token and logit.
    void epilogue(HypTopKSample* d_out, bool draw = false);
    // Capture one decode step of `st` (embed cur's token at *pos, every layer, the head,
    // the sample into cur, pos += 1) as a graph; `draw`: the sampled epilogue.
    GraphExec capture_step(DecoderState& st, bool draw);

    Geometry geo_;
    ModelWeights w_;
    hipStream_t stream_ = nullptr;
    float embed_scale_ = 0.0f;   // bf16(sqrt(hidden)) (forward.cc:103,126-131)
    float softcap_ = 0.0f;       // bf16(final_logit_softcapping)
    DeviceBuffer ids_;           // uint32 [kChunkTokens]
    DeviceBuffer x_, xn_, q_, k_, v_, attn_, o_, h_, d_, last_, logits_;
    DeviceBuffer xr_;            // [kSkinnyMaxM][hidden]: the residual stream's second buffer at decode sizes
    DeviceBuffer attn_ws_, sample_ws_;
    DeviceBuffer stoch_ws_;      // the temperature draw's bins (zero between draws) and SampleParams
    // RoPE (cos, sin) of every position per layer kind, computed once on the device with
    // the rope kernel's arithmetic (a 12B at 262144 positions: 0.8 GB); empty when larger
    // than kRopeTableMaxBytes, then the prepare kernel computes them per token.
    DeviceBuffer rope_local_, rope_global_;
};

constexpr size_t kRopeTableMaxBytes = size_t{4} << 30;

}  // namespace hyperion::model
