// The decoder around the Q4 projections; see decoder.h for what each part replaces.
#include "decoder.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>

#include "kernels.h"
#include "sampling.h"

namespace hyperion::model {

using hip::NativeError;

namespace {

[[noreturn]] void invalid(const std::string& what) { throw NativeError(HYP_STATUS_INVALID_ARGUMENT, what); }
[[noreturn]] void unsupported(const std::string& what) { throw NativeError(HYP_STATUS_UNSUPPORTED, what); }

float host_round_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return f;
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    float r;
    std::memcpy(&r, &u, 4);
    return r;
}

RopeParams rope_from_abi(const HypRopeSpec& s) {
    RopeParams r;
    r.theta = s.theta;
    r.has_partial = s.has_partial_rotary_factor != 0;
    r.partial = s.partial_rotary_factor;
    r.proportional = s.proportional != 0;
    return r;
}

bool attention_head_dim(uint32_t d) { return d == 64u || d == 128u || d == 256u || d == 512u; }

uint16_t* u16(const DeviceBuffer& b) { return static_cast<uint16_t*>(b.data()); }

}  // namespace

Geometry Geometry::from_abi(const HypGeometryParams& p) {
    // Geometry::from_abi (geometry.cc:23-76).
    if (p.layer_types == nullptr && p.num_hidden_layers > 0) invalid("layer_types pointer is null");
    if (p.model_type != HYP_GEMMA4_TEXT && p.model_type != HYP_GEMMA4_UNIFIED_TEXT) {
        invalid("unknown HypTextModelType");
    }
    Geometry g;
    g.types.reserve(p.num_hidden_layers);
    for (uint32_t i = 0; i < p.num_hidden_layers; ++i) {
        if (p.layer_types[i] == HYP_LAYER_SLIDING) {
            g.types.push_back(LayerType::Sliding);
        } else if (p.layer_types[i] == HYP_LAYER_FULL) {
            g.types.push_back(LayerType::Full);
        } else {
            invalid("unknown HypLayerType at index " + std::to_string(i));
        }
    }
    g.hidden = p.hidden_size;
    g.intermediate = p.intermediate_size;
    g.heads = p.num_attention_heads;
    g.head_dim_local = p.head_dim_local;
    g.head_dim_global = p.head_dim_global;
    g.kv_heads_local = p.num_kv_heads_local;
    g.kv_heads_global = p.num_kv_heads_global;
    g.k_eq_v_global = p.attention_k_eq_v_global != 0;
    g.window = p.sliding_window;
    g.rope_local = rope_from_abi(p.rope_local);
    g.rope_global = rope_from_abi(p.rope_global);
    g.softcap = p.final_logit_softcapping;
    g.eps = p.rms_norm_eps;
    g.vocab = p.vocab_size;
    g.max_positions = p.max_position_embeddings;

    // Geometry::validate (geometry.cc:78-130).
    if (g.types.empty()) invalid("layer_types is empty");
    if (g.types.back() != LayerType::Full) invalid("the last layer must be full_attention (Gemma 4 invariant)");
    if (g.window == 0) invalid("sliding_window must be non-zero");
    if (p.num_kv_shared_layers > p.num_hidden_layers) invalid("num_kv_shared_layers exceeds num_hidden_layers");
    if (g.head_dim_local == 0 || g.head_dim_global == 0) {
        invalid("head_dim_local and head_dim_global must be non-zero");
    }
    if (g.heads == 0 || g.kv_heads_local == 0 || g.kv_heads_global == 0) {
        invalid("attention/KV head counts must be non-zero");
    }
    if (g.vocab == 0) invalid("vocab_size must be non-zero");
    if (g.rope_local.proportional) invalid("sliding rope must be the default (full rotary) scheme");
    if (g.rope_local.has_partial) invalid("sliding rope must be full rotary (no partial_rotary_factor)");
    if (!g.rope_global.proportional) invalid("global rope must be the proportional scheme");
    if (!g.rope_global.has_partial) invalid("global rope must set partial_rotary_factor");
    if (!(g.rope_local.theta > 0.0) || !(g.rope_global.theta > 0.0)) invalid("rope_theta must be positive");
    if (p.tie_word_embeddings == 0) {
        invalid("tie_word_embeddings must be true (lm_head is tied to the embedding table)");
    }
    if (p.has_moe != 0 && (p.moe.num_experts == 0 || p.moe.top_k == 0 || p.moe.moe_intermediate_size == 0)) {
        invalid("moe block requires non-zero num_experts/top_k/moe_intermediate_size");
    }
    if (!(g.eps >= 0.0f) || !std::isfinite(g.eps)) invalid("rms_norm_eps must be finite and >= 0");
    if (!(g.softcap > 0.0f) || !std::isfinite(g.softcap)) invalid("final_logit_softcapping must be finite and > 0");
    if (g.max_positions == 0) invalid("max_position_embeddings must be non-zero");

    // What this build runs: the dense Gemma 4 text decoder of the tiny fixture and the 12B.
    if (p.has_moe != 0) unsupported("mixture-of-experts blocks are not built");
    if (p.ple_hidden_per_layer_input != 0 || p.ple_vocab_per_layer_input != 0) {
        unsupported("per-layer input embeddings are not built");
    }
    if (p.use_double_wide_mlp != 0) unsupported("the double-wide MLP is not built");
    if (p.num_kv_shared_layers != 0) unsupported("shared KV layers are not built");
    if (p.attention_bias != 0) unsupported("attention bias is not built");
    if (!g.k_eq_v_global) unsupported("global layers without attention_k_eq_v are not built");
    if (!attention_head_dim(g.head_dim_local) || !attention_head_dim(g.head_dim_global)) {
        unsupported("head dims must be 64, 128, 256 or 512");
    }
    if (g.heads % g.kv_heads_local != 0 || g.heads % g.kv_heads_global != 0) {
        invalid("num_attention_heads must be a multiple of the KV head counts");
    }
    if (g.hidden == 0 || g.hidden % 64u != 0 || g.hidden > hip::residual_norm_max_hidden()) {
        unsupported("hidden_size must be a non-zero multiple of 64, at most 16384");
    }
    if (g.intermediate == 0 || g.intermediate % 64u != 0) {
        unsupported("intermediate_size must be a non-zero multiple of 64");
    }
    const uint32_t rotated = g.rotated_dims(LayerType::Full);
    if (!(g.rope_global.partial > 0.0f) || rotated == 0) invalid("partial_rotary_factor leaves no rotated dims");
    if (rotated > g.head_dim_global) invalid("partial_rotary_factor must be at most 1");
    return g;
}

uint32_t Geometry::rotated_dims(LayerType kind) const noexcept {
    if (kind == LayerType::Sliding) return head_dim_local;
    // Rope::Rope (rope.cc:44-49): floor(prf * head_dim) in fp32, rounded down to even.
    const float r = rope_global.partial * static_cast<float>(head_dim_global);
    if (!(r >= 0.0f)) return 0;
    uint32_t rotated = r >= 4294967295.0f ? 0xffffffffu : static_cast<uint32_t>(r);
    rotated -= rotated % 2u;
    return rotated;
}

namespace {

// The tiled resident allocation of one [n, k] projection (qlinear.cc make_storage).
uint64_t q4_resident_bytes(uint64_t n, uint64_t k) {
    const uint64_t tiles = (n + 15u) / 16u;
    const uint64_t pairs = (k + 127u) / 128u;
    const auto a256 = [](uint64_t v) { return (v + 255u) & ~uint64_t{255u}; };
    return a256(tiles * pairs * 1024u) + a256(tiles * pairs * 128u);
}

uint32_t cache_capacity(const Geometry& g, LayerType kind) {
    return kind == LayerType::Sliding ? std::min(g.window + kChunkTokens, g.max_positions) : g.max_positions;
}

uint64_t rope_table_bytes(const Geometry& g, uint32_t D) {
    const uint64_t bytes = static_cast<uint64_t>(g.max_positions) * (D / 2u) * sizeof(float2);
    return bytes > kRopeTableMaxBytes ? 0u : bytes;
}

// The attention split workspace: decode splits, and the chunk form's two key splits up to
// one prefill chunk, for both layer kinds.
uint64_t attention_ws_bytes(const Geometry& g) {
    const uint32_t chunk = std::min(kChunkTokens, g.max_positions);
    return std::max({hip::attention_workspace_bytes(g.kv_heads_local, g.head_dim_local),
                     hip::attention_workspace_bytes(g.kv_heads_global, g.head_dim_global),
                     hip::attention_chunk_workspace_bytes(chunk, g.heads, g.kv_heads_local, g.head_dim_local),
                     hip::attention_chunk_workspace_bytes(chunk, g.heads, g.kv_heads_global, g.head_dim_global)});
}

}  // namespace

MemoryReport plan_memory(const Geometry& g) {
    MemoryReport r;
    const uint64_t H = g.heads;
    auto proj = [&](uint64_t n, uint64_t k) {
        r.weight_bytes += q4_resident_bytes(n, k);
        r.dense_bf16_weight_bytes += 2u * n * k;
    };
    proj(g.vocab, g.hidden);   // the embedding, tied as the LM head
    for (LayerType kind : g.types) {
        const bool sliding = kind == LayerType::Sliding;
        const uint64_t D = sliding ? g.head_dim_local : g.head_dim_global;
        const uint64_t kvh = sliding ? g.kv_heads_local : g.kv_heads_global;
        proj(H * D, g.hidden);
        proj(kvh * D, g.hidden);
        if (sliding) proj(kvh * D, g.hidden);
        proj(g.hidden, H * D);
        proj(g.intermediate, g.hidden);
        proj(g.intermediate, g.hidden);
        proj(g.hidden, g.intermediate);
        r.norm_bytes += 2u * (4u * g.hidden + 2u * D + 1u);
        const uint64_t kv = 2u * static_cast<uint64_t>(cache_capacity(g, kind)) * kvh * D * 2u;
        (sliding ? r.kv_local_bytes : r.kv_global_bytes) += kv;
    }
    r.norm_bytes += 2u * g.hidden;
    r.state_bytes = sizeof(HypTopKSample) + 2u * sizeof(uint32_t);
    const uint64_t T = kChunkTokens;
    const uint64_t dmax = std::max(g.head_dim_local, g.head_dim_global);
    const uint64_t kvmax = std::max(g.kv_heads_local * g.head_dim_local, g.kv_heads_global * g.head_dim_global);
    r.scratch_bytes = T * 4u + 4u * T * g.hidden * 2u + 2u * T * H * dmax * 2u + 2u * T * kvmax * 2u +
                      T * g.intermediate * 2u + static_cast<uint64_t>(g.hidden) * 2u +
                      uint64_t{hip::kSkinnyMaxM} * g.hidden * 2u + static_cast<uint64_t>(g.vocab) * 2u +
                      attention_ws_bytes(g) +
                      hip::sample_greedy_workspace_bytes() + hip::sample_stochastic_workspace_bytes() +
                      rope_table_bytes(g, g.head_dim_local) +
                      rope_table_bytes(g, g.head_dim_global);
    return r;
}

MemoryReport Decoder::memory() const {
    MemoryReport r;
    auto lin = [&](const QuantizedLinear& q) {
        r.weight_bytes += q.storage.bytes();
        r.dense_bf16_weight_bytes += 2u * static_cast<uint64_t>(q.mat.n) * q.mat.k;
    };
    lin(w_.embed);
    for (const LayerWeights& lw : w_.layers) {
        lin(lw.q_proj);
        lin(lw.k_proj);
        if (lw.v_proj) lin(*lw.v_proj);
        lin(lw.o_proj);
        lin(lw.gate_proj);
        lin(lw.up_proj);
        lin(lw.down_proj);
        for (const DeviceBuffer& b : lw.norms) r.norm_bytes += b.bytes();
    }
    r.norm_bytes += w_.final_norm.bytes();
    for (const DeviceBuffer* b : {&ids_, &x_, &xn_, &xr_, &q_, &k_, &v_, &attn_, &o_, &h_, &d_, &last_, &logits_, &attn_ws_,
                                  &sample_ws_, &stoch_ws_, &rope_local_, &rope_global_}) {
        r.scratch_bytes += b->bytes();
    }
    const MemoryReport planned = plan_memory(geo_);   // a state is not allocated to be counted
    r.kv_local_bytes = planned.kv_local_bytes;
    r.kv_global_bytes = planned.kv_global_bytes;
    r.state_bytes = planned.state_bytes;
    return r;
}

GraphExec::~GraphExec() {
    if (exec_ != nullptr) (void)hipGraphExecDestroy(exec_);
}

GraphExec& GraphExec::operator=(GraphExec&& o) noexcept {
    if (this != &o) {
        if (exec_ != nullptr) (void)hipGraphExecDestroy(exec_);
        exec_ = o.exec_;
        o.exec_ = nullptr;
    }
    return *this;
}

Decoder::Decoder(Geometry geometry, ModelWeights weights) : geo_(std::move(geometry)), w_(std::move(weights)) {
    const Geometry& g = geo_;
    if (!w_.has_norms) invalid("the weights artifact is missing norm vectors or layer scalars");
    if (w_.layers.size() != g.types.size()) {
        invalid("the artifact holds " + std::to_string(w_.layers.size()) + " layers, the geometry " +
                std::to_string(g.types.size()));
    }
    // The weight schema must agree with the geometry (weights_loader.cc:116-124), and every
    // tensor with its dims (weights_test.cc:76-82 checks the same on the fixture).
    if (w_.embed.mat.n != g.vocab || w_.embed.mat.k != g.hidden) invalid("embed_tokens is not [vocab, hidden]");
    if (w_.final_norm_len != g.hidden) invalid("the final norm is not [hidden]");
    for (size_t i = 0; i < w_.layers.size(); ++i) {
        const LayerWeights& lw = w_.layers[i];
        const std::string at = "layer " + std::to_string(i) + ": ";
        if (lw.kind != g.types[i]) {
            invalid(at + "weight schema (" + (lw.kind == LayerType::Sliding ? "sliding" : "global") +
                    ") disagrees with geometry layer_types");
        }
        const bool sliding = lw.kind == LayerType::Sliding;
        const uint32_t D = sliding ? g.head_dim_local : g.head_dim_global;
        const uint32_t kvh = sliding ? g.kv_heads_local : g.kv_heads_global;
        auto shape = [&](const QuantizedLinear& l, uint32_t n, uint32_t k, const char* name) {
            if (l.mat.n != n || l.mat.k != k) {
                invalid(at + name + " is [" + std::to_string(l.mat.n) + ", " + std::to_string(l.mat.k) +
                        "], expected [" + std::to_string(n) + ", " + std::to_string(k) + "]");
            }
        };
        shape(lw.q_proj, g.heads * D, g.hidden, "q_proj");
        shape(lw.k_proj, kvh * D, g.hidden, "k_proj");
        if (sliding) shape(*lw.v_proj, kvh * D, g.hidden, "v_proj");
        shape(lw.o_proj, g.hidden, g.heads * D, "o_proj");
        shape(lw.gate_proj, g.intermediate, g.hidden, "gate_proj");
        shape(lw.up_proj, g.intermediate, g.hidden, "up_proj");
        shape(lw.down_proj, g.hidden, g.intermediate, "down_proj");
        const uint32_t want[kLayerNorms] = {g.hidden, g.hidden, g.hidden, g.hidden, D, D, 1u};
        for (int j = 0; j < kLayerNorms; ++j) {
            if (lw.norm_len[j] != want[j]) invalid(at + "a norm vector or layer_scalar has the wrong length");
        }
    }

    embed_scale_ = host_round_bf16(std::sqrt(static_cast<float>(g.hidden)));
    softcap_ = host_round_bf16(g.softcap);
    HYP_HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));

    const size_t T = kChunkTokens;
    const uint32_t dmax = std::max(g.head_dim_local, g.head_dim_global);
    const uint32_t kvmax = std::max(g.kv_heads_local * g.head_dim_local, g.kv_heads_global * g.head_dim_global);
    ids_ = DeviceBuffer(T * sizeof(uint32_t));
    x_ = DeviceBuffer(T * g.hidden * 2u);
    xn_ = DeviceBuffer(T * g.hidden * 2u);
    xr_ = DeviceBuffer(size_t{hip::kSkinnyMaxM} * g.hidden * 2u);
    q_ = DeviceBuffer(T * g.heads * dmax * 2u);
    k_ = DeviceBuffer(T * kvmax * 2u);
    v_ = DeviceBuffer(T * kvmax * 2u);
    attn_ = DeviceBuffer(T * g.heads * dmax * 2u);
    o_ = DeviceBuffer(T * g.hidden * 2u);
    h_ = DeviceBuffer(T * g.intermediate * 2u);
    d_ = DeviceBuffer(T * g.hidden * 2u);
    last_ = DeviceBuffer(static_cast<size_t>(g.hidden) * 2u);
    logits_ = DeviceBuffer(static_cast<size_t>(g.vocab) * 2u);
    attn_ws_ = DeviceBuffer(attention_ws_bytes(g));
    sample_ws_ = DeviceBuffer(hip::sample_greedy_workspace_bytes());
    stoch_ws_ = DeviceBuffer(hip::sample_stochastic_workspace_bytes());
    hip::init_sample_stochastic_workspace(stoch_ws_.data(), stream_);
    const auto table = [&](uint32_t D, LayerType kind, double theta) {
        const size_t bytes = rope_table_bytes(g, D);
        if (bytes == 0) return DeviceBuffer();
        DeviceBuffer t(bytes);
        hip::launch_rope_table(static_cast<float2*>(t.data()), g.max_positions, D, g.rotated_dims(kind),
                               static_cast<float>(theta), stream_);
        return t;
    };
    rope_local_ = table(g.head_dim_local, LayerType::Sliding, g.rope_local.theta);
    rope_global_ = table(g.head_dim_global, LayerType::Full, g.rope_global.theta);
    HYP_HIP_CHECK(hipStreamSynchronize(stream_));
}

Decoder::~Decoder() {
    if (stream_ != nullptr) {
        (void)hipStreamSynchronize(stream_);
        (void)hipStreamDestroy(stream_);
    }
}

DecoderState Decoder::make_state() const {
    const Geometry& g = geo_;
    DecoderState st;
    st.caches.reserve(g.types.size());
    for (LayerType kind : g.types) {
        LayerCache c;
        const bool sliding = kind == LayerType::Sliding;
        c.head_dim = sliding ? g.head_dim_local : g.head_dim_global;
        c.kv_heads = sliding ? g.kv_heads_local : g.kv_heads_global;
        c.cap = cache_capacity(g, kind);
        const size_t bytes = static_cast<size_t>(c.cap) * c.kv_heads * c.head_dim * 2u;
        c.k = DeviceBuffer(bytes);
        c.v = DeviceBuffer(bytes);
        // Unwritten slots are never read (the masks stop at the committed positions), but
        // cleared memory keeps a stray read finite.
        HYP_HIP_CHECK(hipMemsetAsync(c.k.data(), 0, bytes, stream_));
        HYP_HIP_CHECK(hipMemsetAsync(c.v.data(), 0, bytes, stream_));
        (sliding ? st.local_bytes : st.global_bytes) += 2u * bytes;
        st.caches.push_back(std::move(c));
    }
    st.cur = DeviceBuffer(sizeof(HypTopKSample));
    st.counters = DeviceBuffer(2u * sizeof(uint32_t));
    HYP_HIP_CHECK(hipMemsetAsync(st.cur.data(), 0, st.cur.bytes(), stream_));
    HYP_HIP_CHECK(hipMemsetAsync(st.counters.data(), 0, st.counters.bytes(), stream_));
    HYP_HIP_CHECK(hipStreamSynchronize(stream_));
    return st;
}

GraphExec Decoder::capture_step(DecoderState& st, bool draw) {
    auto* cur = static_cast<HypTopKSample*>(st.cur.data());
    auto* counters = static_cast<uint32_t*>(st.counters.data());
    HYP_HIP_CHECK(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
    hipGraph_t graph = nullptr;
    try {
        forward_chunk(st, &cur->token_id, 1, 0, nullptr, counters);
        epilogue(cur, draw);
        hip::launch_decode_advance(counters, counters + 1, cur, stream_);
    } catch (...) {
        (void)hipStreamEndCapture(stream_, &graph);
        if (graph != nullptr) (void)hipGraphDestroy(graph);
        throw;
    }
    HYP_HIP_CHECK(hipStreamEndCapture(stream_, &graph));
    hipGraphExec_t exec = nullptr;
    const hipError_t err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    HYP_HIP_CHECK(err);
    return GraphExec(exec);
}

void Decoder::forward_chunk(DecoderState& st, const uint32_t* d_ids, uint32_t L, uint32_t offset,
                            uint16_t* final_rows, const uint32_t* d_pos) {
    const Geometry& g = geo_;
    hipStream_t s = stream_;
    uint16_t* x = u16(x_);
    uint16_t* xn = u16(xn_);
    const float eps = g.eps;
    // At decode sizes the q/k/v launch normalises its input rows itself (the same bits as
    // the standalone norm); above them the input norm is a pass of its own, fused into the
    // previous layer's closing residual kernel.
    const bool norm_in_qkv = L <= hip::kSkinnyMaxM && hip::skinny_norm_supported(L, g.hidden);
    // And a layer's closing residual update (x + rms(d) * w_post_ff, times the layer
    // scalar) runs in the prologue of the next layer's q/k/v launch, which writes the
    // updated stream to the other of two buffers (x_, xr_); the last layer's close is a
    // residual kernel that also forms the final norm. Same bits as the separate kernels.
    // (In the fused gate/up's prologue the attention half's close measured slower than its
    // own kernel: that launch runs about two rounds of workgroups, each paying it.)
    const bool fuse_residual = norm_in_qkv && hip::skinny_resid_supported(L, g.hidden);
    uint16_t* other = u16(xr_);   // fuse_residual: the buffer the next prologue writes

    // ForwardPass::embed (forward.cc:126-131): gathered rows dequantized, times bf16(sqrt(hidden)).
    hip::launch_q4_dequantize_tiled(w_.embed.mat, d_ids, L, embed_scale_, x, s);
    if (!norm_in_qkv) {
        hip::launch_rms_normalize(x, w_.layers[0].norm(LayerNorm::kInput), L, g.hidden, eps, xn, s);
    }

    for (size_t i = 0; i < w_.layers.size(); ++i) {
        const LayerWeights& lw = w_.layers[i];
        LayerCache& cache = st.caches[i];
        const bool sliding = lw.kind == LayerType::Sliding;
        const uint32_t D = cache.head_dim;
        const uint32_t kvh = cache.kv_heads;

        // q/k/v (forward.cc:395-409; a global layer has no v_proj: K = V).
        const hip::Q4Matrix* ws[3] = {&lw.q_proj.mat, &lw.k_proj.mat, sliding ? &lw.v_proj->mat : nullptr};
        uint16_t* ys[3] = {u16(q_), u16(k_), u16(v_)};
        const uint32_t count = sliding ? 3u : 2u;
        if (fuse_residual && i > 0) {
            const LayerWeights& prev = w_.layers[i - 1];
            const hip::SkinnyResidual res{u16(d_), x, other, prev.norm(LayerNorm::kPostFeedforward),
                                          prev.norm(LayerNorm::kScalar)};
            hip::launch_q4_skinny_group(ws, ys, count, x, L, &eps, lw.norm(LayerNorm::kInput), s, &res);
            std::swap(x, other);
        } else if (norm_in_qkv) {
            hip::launch_q4_skinny_group(ws, ys, count, x, L, &eps, lw.norm(LayerNorm::kInput), s);
        } else if (hip::skinny_supported(L, g.hidden, false)) {
            hip::launch_q4_skinny_group(ws, ys, count, xn, L, nullptr, nullptr, s);
        } else {
            hip::launch_q4_gemm_group(ws, ys, count, xn, L, s);
        }

        // q_norm / k_norm / v_norm, RoPE, the cache append (forward.cc:400-459).
        hip::AttnPrepareArgs pa{};
        pa.pos = d_pos;
        pa.rope_cs = static_cast<const float2*>((sliding ? rope_local_ : rope_global_).data());
        pa.q = u16(q_);
        pa.k_raw = u16(k_);
        pa.v_raw = sliding ? u16(v_) : nullptr;
        pa.q_norm = lw.norm(LayerNorm::kQ);
        pa.k_norm = lw.norm(LayerNorm::kK);
        pa.cache_k = u16(cache.k);
        pa.cache_v = u16(cache.v);
        pa.L = L;
        pa.n_heads = g.heads;
        pa.n_kv_heads = kvh;
        pa.head_dim = D;
        pa.rotated = g.rotated_dims(lw.kind);
        pa.offset = offset;
        pa.cap = cache.cap;
        pa.base = static_cast<float>(sliding ? g.rope_local.theta : g.rope_global.theta);
        pa.eps = eps;
        // One token (a decode step) with the RoPE table: the attention launch does this
        // work itself (the same bits), one launch fewer per layer.
        const bool fold_prepare = L == 1u && pa.rope_cs != nullptr && hip::attention_prep_fits(g.heads, kvh, D);
        if (!fold_prepare) hip::launch_attn_prepare(pa, s);

        // SDPA over the visible cached prefix and the appended chunk (forward.cc:420-505).
        hip::AttnArgs aa{};
        aa.q = u16(q_);
        aa.k = nullptr;
        aa.v = nullptr;
        aa.cache_k = u16(cache.k);
        aa.cache_v = u16(cache.v);
        aa.out = u16(attn_);
        aa.L = L;
        aa.n_heads = g.heads;
        aa.n_kv_heads = kvh;
        aa.head_dim = D;
        aa.cap = cache.cap;
        aa.offset = offset;
        aa.prefix_len = sliding ? std::min(g.window, offset) : offset;
        aa.window = sliding ? g.window : 0u;
        aa.workspace = attn_ws_.data();
        aa.workspace_bytes = attn_ws_.bytes();
        if (d_pos != nullptr) {
            // Splits sized for the longest key range the replays can see.
            const uint32_t max_keys = sliding ? std::min(g.window, g.max_positions) + L : g.max_positions;
            aa.pos = d_pos;
            aa.fixed_splits = hip::attention_splits(L, g.heads, kvh, max_keys);
        }
        if (fold_prepare) aa.prep = &pa;
        hip::launch_attention(aa, s);

        // o, then the attention half of the sandwich and the MLP's input norm (forward.cc:518-526).
        lw.o_proj.apply(u16(attn_), L, u16(o_), s);
        hip::launch_residual_norm(u16(o_), x, lw.norm(LayerNorm::kPostAttention), nullptr,
                                  lw.norm(LayerNorm::kPreFeedforward), xn, L, g.hidden, eps, s);
        // mlp (forward.cc:338-343), the feed-forward half and the layer scalar (:527-539).
        mlp_gate_up(lw.gate_proj, lw.up_proj, xn, L, u16(h_), s);
        lw.down_proj.apply(u16(h_), L, u16(d_), s);
        if (fuse_residual) {
            if (i + 1 < w_.layers.size()) continue;   // closed by the next layer's q/k/v launch
            // The last close, with final_norm (forward.cc:133-135) as its next norm.
            const uint16_t* fw = static_cast<const uint16_t*>(w_.final_norm.data());
            uint16_t* fin = final_rows != nullptr ? final_rows : (L == 1u ? u16(last_) : nullptr);
            hip::launch_residual_norm(u16(d_), x, lw.norm(LayerNorm::kPostFeedforward), lw.norm(LayerNorm::kScalar),
                                      fin != nullptr ? fw : nullptr, fin, L, g.hidden, eps, s);
            if (fin == nullptr) {
                hip::launch_rms_normalize(x + static_cast<size_t>(L - 1) * g.hidden, fw, 1, g.hidden, eps,
                                          u16(last_), s);
            }
            return;
        }
        const uint16_t* next_w =
            !norm_in_qkv && i + 1 < w_.layers.size() ? w_.layers[i + 1].norm(LayerNorm::kInput) : nullptr;
        hip::launch_residual_norm(u16(d_), x, lw.norm(LayerNorm::kPostFeedforward), lw.norm(LayerNorm::kScalar),
                                  next_w, next_w != nullptr ? xn : nullptr, L, g.hidden, eps, s);
    }

    // final_norm (forward.cc:133-135).
    const uint16_t* fw = static_cast<const uint16_t*>(w_.final_norm.data());
    if (final_rows != nullptr) {
        hip::launch_rms_normalize(x, fw, L, g.hidden, eps, final_rows, s);
    } else {
        hip::launch_rms_normalize(x + static_cast<size_t>(L - 1) * g.hidden, fw, 1, g.hidden, eps, u16(last_), s);
    }
}

void Decoder::epilogue(HypTopKSample* d_out, bool draw) {
    // run_epilogue (model.cc:215-228): tied lm_head + softcap on the last position, then
    // the greedy pick with its top-k sidecar (model.cc:262-288). The sampled epilogue
    // (model.cc:262-301) keeps that sidecar of the pre-filter logits (forward.cc:303-319) and
    // replaces the token with the draw.
    w_.embed.apply(u16(last_), 1, u16(logits_), stream_, Epilogue::kSoftcap, softcap_);
    hip::launch_sample_topk(u16(logits_), 1, geo_.vocab, d_out, sample_ws_.data(), sample_ws_.bytes(), stream_);
    if (draw) {
        hip::launch_sample_stochastic(u16(logits_), geo_.vocab, stoch_ws_.data(), stoch_ws_.bytes(), d_out, stream_);
    }
}

void Decoder::forward_hidden(DecoderState& st, const uint32_t* ids, uint32_t count, uint32_t offset,
                             uint16_t* hidden_out) {
    const Geometry& g = geo_;
    if (count == 0) invalid("forward requires at least one token");
    if (static_cast<uint64_t>(offset) + count > g.max_positions) invalid("positions exceed max_position_embeddings");
    for (uint32_t i = 0; i < count; ++i) {
        if (ids[i] >= g.vocab) invalid("token id " + std::to_string(ids[i]) + " is outside the vocabulary");
    }
    for (uint32_t done = 0; done < count;) {
        const uint32_t take = std::min(kChunkTokens, count - done);
        HYP_HIP_CHECK(hipMemcpyAsync(ids_.data(), ids + done, take * sizeof(uint32_t), hipMemcpyHostToDevice, stream_));
        forward_chunk(st, static_cast<const uint32_t*>(ids_.data()), take, offset + done, u16(o_));
        HYP_HIP_CHECK(hipMemcpyAsync(hidden_out + static_cast<size_t>(done) * g.hidden, o_.data(),
                                     static_cast<size_t>(take) * g.hidden * 2u, hipMemcpyDeviceToHost, stream_));
        HYP_HIP_CHECK(hipStreamSynchronize(stream_));
        done += take;
    }
}

StepSample Decoder::prefill(DecoderState& st, const uint32_t* ids, uint32_t count,
                            const HypSamplingConfig* sampling) {
    const Geometry& g = geo_;
    if (st.offset != 0) invalid("prefill requires a fresh (offset 0) KV state");
    if (count > g.max_positions) invalid("the prompt exceeds max_position_embeddings");
    for (uint32_t i = 0; i < count; ++i) {
        if (ids[i] >= g.vocab) invalid("token id " + std::to_string(ids[i]) + " is outside the vocabulary");
    }
    auto* cur = static_cast<HypTopKSample*>(st.cur.data());
    for (uint32_t done = 0; done < count;) {
        const uint32_t take = std::min(kChunkTokens, count - done);
        HYP_HIP_CHECK(hipMemcpyAsync(ids_.data(), ids + done, take * sizeof(uint32_t), hipMemcpyHostToDevice, stream_));
        forward_chunk(st, static_cast<const uint32_t*>(ids_.data()), take, done, nullptr);
        done += take;
        if (done == count) {
            if (sampling != nullptr) {
                // The prefill's draw uses the request seed itself (model.cc:840-841).
                const hip::SampleParams p = sampling_params(*sampling);
                hip::launch_sample_params(stoch_ws_.data(), p.inv_temp, p.top_p, p.min_p, p.top_k,
                                          sampling_uniform(sampling->seed), stream_);
            }
            epilogue(cur, sampling != nullptr);
        }
        // The ids buffer is reused by the next chunk: its copy waits for this chunk.
        HYP_HIP_CHECK(hipStreamSynchronize(stream_));
    }
    StepSample out;
    HYP_HIP_CHECK(hipMemcpy(&out.sample, cur, sizeof(HypTopKSample), hipMemcpyDeviceToHost));
    out.near_tie_events = out.sample.near_tie != 0u ? 1u : 0u;
    st.offset = count;
    st.last_token = out.sample.token_id;
    return out;
}

namespace {

// Marks a DecoderState consumed unless disarmed: armed once a decode's first replay is
// enqueued (the replays advance the live KV rows, cursor and token in place), disarmed when
// the block has completed and `offset` agrees with the device (DirectKvExecutionGuard,
// model.cc:79-105). On the failure path it also waits for the stream, so that no replay still
// reads the state's buffers when the caller frees it.
class ConsumeOnFailure {
  public:
    ConsumeOnFailure(DecoderState& st, hipStream_t stream) noexcept : st_(st), stream_(stream) {}
    ConsumeOnFailure(const ConsumeOnFailure&) = delete;
    ConsumeOnFailure& operator=(const ConsumeOnFailure&) = delete;
    ~ConsumeOnFailure() {
        if (armed_) {
            st_.consumed = true;
            (void)hipStreamSynchronize(stream_);
        }
    }
    void arm() noexcept { armed_ = true; }
    void disarm() noexcept { armed_ = false; }

  private:
    DecoderState& st_;
    hipStream_t stream_;
    bool armed_ = false;
};

#ifdef HYP_TEST_FAULTS
// Test builds only (libhyperion_hip_faults.so): a one-shot host-side throw right after a
// decode's first replay is enqueued, as the reference's test build injects a failure into its
// forward (test_fault.cc, forward.cc:564-566). No GPU work is affected.
thread_local bool g_fault_after_first_replay = false;
#endif

}  // namespace

StepSample Decoder::decode(DecoderState& st, uint32_t n_tokens, const HypSamplingConfig* sampling) {
    const Geometry& g = geo_;
    if (st.offset == 0) invalid("decode requires a populated KV state (prefill first)");
    if (static_cast<uint64_t>(st.offset) + n_tokens > g.max_positions) {
        invalid("decoding past max_position_embeddings");
    }
    StepSample out;
    if (n_tokens == 0) return out;
    GraphExec& graph = sampling != nullptr ? st.sampled_step : st.step;
    if (graph.get() == nullptr) graph = capture_step(st, sampling != nullptr);
    // The draws' parameters: per block of up to kMaxSampledSteps replays, the config and
    // the uniform of each step's RNG state (the state starts at the seed every call and
    // advances per step, model.cc:926-944). Each block's copy is queued before its replays;
    // the host blocks stay alive until the stream has been synchronised below.
    std::vector<hip::SampleParams> blocks;
    if (sampling != nullptr) {
        blocks.resize((n_tokens + hip::kMaxSampledSteps - 1u) / hip::kMaxSampledSteps, sampling_params(*sampling));
        uint64_t state = sampling->seed;
        for (uint32_t j = 0; j < n_tokens; ++j) {
            hip::SampleParams& b = blocks[j / hip::kMaxSampledSteps];
            b.uniform[b.n_uniform++] = sampling_uniform(state);
            state = advance_sampling_state(state);
        }
    }
    hip::SampleParams* d_params = hip::sample_stochastic_params(stoch_ws_.data());
    // The replays start from the cursor with a cleared near-tie count; each embeds the
    // token in cur, samples the next one into cur and advances the position.
    const uint32_t start[2] = {st.offset, 0u};
    auto* counters = static_cast<uint32_t*>(st.counters.data());
    HYP_HIP_CHECK(hipMemcpyAsync(counters, start, sizeof(start), hipMemcpyHostToDevice, stream_));
    ConsumeOnFailure guard(st, stream_);
    guard.arm();
    for (uint32_t j = 0; j < n_tokens; ++j) {
        if (sampling != nullptr && j % hip::kMaxSampledSteps == 0u) {
            HYP_HIP_CHECK(hipMemcpyAsync(d_params, &blocks[j / hip::kMaxSampledSteps], sizeof(hip::SampleParams),
                                         hipMemcpyHostToDevice, stream_));
        }
        HYP_HIP_CHECK(hipGraphLaunch(graph.get(), stream_));
#ifdef HYP_TEST_FAULTS
        if (g_fault_after_first_replay) {
            g_fault_after_first_replay = false;
            throw std::runtime_error("injected failure after the first decode replay");
        }
#endif
    }
    uint32_t end[2] = {0u, 0u};
    HYP_HIP_CHECK(hipMemcpyAsync(&out.sample, st.cur.data(), sizeof(HypTopKSample), hipMemcpyDeviceToHost, stream_));
    HYP_HIP_CHECK(hipMemcpyAsync(end, counters, sizeof(end), hipMemcpyDeviceToHost, stream_));
    HYP_HIP_CHECK(hipStreamSynchronize(stream_));
    HYP_REQUIRE(end[0] == st.offset + n_tokens, HYP_STATUS_INTERNAL, "decode: the device position did not advance");
    out.near_tie_events = end[1];
    st.offset += n_tokens;
    st.last_token = out.sample.token_id;
    guard.disarm();
    return out;
}

}  // namespace hyperion::model

#ifdef HYP_TEST_FAULTS
extern "C" void hyp_test_fault_after_first_replay(void) {
    hyperion::model::g_fault_after_first_replay = true;
}
#endif
