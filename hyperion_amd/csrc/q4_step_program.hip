// Persistent decode-step program on gfx950: the ops of step_program.h (q/k/v with the
// rms prologue, o, the fused gate/up GELU, down, ... for every layer) run in ONE launch of
// one 16-wave workgroup per compute unit, instead of one launch per op.
//
// Replaces the per-token layer loop of the reference's decode (ForwardPass::forward,
// native/hyperion_mlx/src/forward.cc:558-563, driven per token by hyp_decode_block,
// model.cc:703-718) for its quantized linears. Each separate launch carries a fixed cost
// of 4-5 us on this part (dispatch, the kernel-boundary cache maintenance, the ramp of the
// first loads); a 12B decode step has 192 of them against ~16 us of weight streaming per
// layer. Here an op boundary costs one round of device-memory counters, and the next op's
// weights are already in flight while it is waited for:
//
//   for each op i:
//     arrive for op i - 1 (this workgroup's outputs of op i - 1 are complete)
//     issue this wave's weight loads for op i (they do not depend on the activations)
//     wait until every workgroup has arrived for op i - 1
//     stage op i's input x into LDS (coherent loads), compute, reduce, store y (coherent)
//
// Coherence across the 8 XCDs (each with its own L2): activations cross workgroups only
// through loads and stores with the system-coherence bits (sc0 sc1, the encoding of a
// system-scope atomic load or store), and a workgroup arrives (a system-scope atomic add)
// only after the waves that stored have waited for their stores to complete. Weights are
// read-only and use the streaming policy as in the per-call kernel.
//
// Every wait is bounded: a workgroup that polls past the spin limit sets the program's
// error word, and every waiting workgroup gives up when it sees it, so the grid always
// drains. The launch is cooperative (all workgroups co-resident, or the launch fails).
//
// The arithmetic of an op is the per-call kernel's (q4_skinny_core.h, q4_rmsnorm.h) with
// the same k splits, so the outputs are the same bits as the per-call entry points.
#include "common.h"
#include "kernels.h"
#include "q4_layout.h"
#include "q4_rmsnorm.h"
#include "q4_skinny_core.h"
#include "step_program.h"

namespace hyperion::hip {
namespace {

constexpr int kCoherent = 17;   // cache policy sc0 | sc1: system coherent

// The op descriptors are read through the constant address space: they do not change
// during a launch, so every field is a scalar load (a generic pointer leaves the compiler
// unable to rule out the kernel's own stores, and it falls back to vector loads).
typedef const __attribute__((address_space(4))) StepOp ConstStepOp;
constexpr uint32_t kThreads = 64u * kStepWaves;

__device__ __forceinline__ uint32_t sys_load(uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// LDS of one op: control words, x rows (WS chunks apart) and a zero row, per-group sums
// of x, the split reduction area, the rms partials (kNorm) and the gate/up combine (kDual).
struct OpLds {
    uint32_t* ctl;
    uint4* xs;
    uint4* zs;
    float4* sx;
    float* red;
    float* part;
    float* comb;
};

template <int M>
__device__ __forceinline__ OpLds op_lds(uint4* smem, uint32_t WS, uint32_t G, bool norm) {
    OpLds l;
    l.ctl = reinterpret_cast<uint32_t*>(smem);
    l.xs = smem + 1;
    l.zs = l.xs + M * WS;
    l.sx = reinterpret_cast<float4*>(l.zs + WS);
    l.red = reinterpret_cast<float*>(l.sx + G);
    l.part = l.red + kStepWaves * M * kTileRows;
    l.comb = l.part + (norm ? M * G + M : 0u);
    return l;
}

// One 64-element unit of x (8 x 16 bytes), read coherently.
__device__ __forceinline__ void load_unit(__amdgpu_buffer_rsrc_t xr, uint32_t off, uint4 (&xv)[8]) {
#pragma unroll
    for (int t = 0; t < 8; ++t)
        xv[t] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16u * t, 0, kCoherent));
}

// Arrive for op `prev`: every wave is past it and the storing waves' outputs are
// complete. Called before the next op's weight loads are issued, so the arrival (a
// vector-memory atomic) does not queue behind them in the compute unit's memory pipeline.
__device__ __forceinline__ void arrive(uint32_t* sync, uint32_t prev, uint32_t tid) {
    // The barrier waits for LDS only (s_waitcnt lgkmcnt(0) on gfx950); its fences keep the
    // compiler from moving the arrival above it.
    __syncthreads();
    if (tid == 0u)
        __hip_atomic_fetch_add(sync + kSyncCounters + (prev * kStepSlots + blockIdx.x % kStepSlots) * kSyncStride, 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Wait until every workgroup has arrived for op `prev`. Returns false when the wait gave up
// (spin limit, or another workgroup's error). The polls queue behind this workgroup's
// weight loads already in flight, so the first one returns about when those have landed.
__device__ __forceinline__ bool wait_all(uint32_t* sync, uint32_t prev, uint32_t target, uint32_t spin_limit,
                                         uint32_t* ctl, uint32_t lane, uint32_t wave) {
    uint32_t* ctr = sync + kSyncCounters + prev * kStepSlots * kSyncStride;
    if (wave == 0u) {
        uint32_t done = 0u;
        for (uint32_t spin = 0;; ++spin) {
            const uint32_t v = lane < kStepSlots ? sys_load(ctr + lane * kSyncStride) : target;
            if (__builtin_amdgcn_ballot_w64(v < target) == 0u) {
                done = 1u;
                break;
            }
            if (spin >= spin_limit) {
                if (lane == 0u)
                    __hip_atomic_store(sync + kSyncError, kStepErrTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                break;
            }
            if (__builtin_amdgcn_readfirstlane(sys_load(sync + kSyncError)) != 0u) break;
            __builtin_amdgcn_s_sleep(2);
        }
        if (lane == 0u) ctl[0] = done;
    }
    __syncthreads();
    return __builtin_amdgcn_readfirstlane(ctl[0]) != 0u;
}

// Stage the op's input rows into LDS as the per-call kernel does (permuted 8-element
// words, per-group sums, the rms prologue with NORM), reading x coherently.
template <int M>
__device__ __forceinline__ void stage_x(ConstStepOp& d, const OpLds& L, bool norm, uint32_t k, uint32_t G, uint32_t WS,
                                        uint32_t tid, uint32_t lane, uint32_t wave) {
    const uint32_t units = M * G;
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(d.x, M * k * 2u);
    uint4 xv[8];
    if (norm) {
        for (uint32_t u = tid; u < units; u += kThreads) {
            const uint32_t m = unit_row<M>(u, G);
            load_unit(xr, (m * k + (u - m * G) * 64u) * 2u, xv);
            L.part[u] = unit_sumsq(xv);
        }
        __syncthreads();
        if (wave < static_cast<uint32_t>(M)) {
            const float ss = row_sumsq(L.part + wave * G, G, lane);
            if (lane == 0u) L.part[units + wave] = rms_inverse(ss, k, d.eps);
        }
        __syncthreads();
    }
    // With at most one unit per thread the rms pass's loads are kept for the staging pass.
    const bool reload = !norm || units > kThreads;
    for (uint32_t u = tid; u < units; u += kThreads) {
        const uint32_t m = unit_row<M>(u, G);
        const uint32_t g = u - m * G;
        if (reload) load_unit(xr, (m * k + g * 64u) * 2u, xv);
        if (norm) {
            normalize_unit(xv, L.part[units + m]);
            if (d.norm_w != nullptr) {
                const uint4* wsrc = reinterpret_cast<const uint4*>(d.norm_w + g * 64u);
                uint4 wv[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) wv[t] = wsrc[t];
                weight_unit(xv, wv);
            }
        }
        float s0 = 0.0f;
        float s1 = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            uint4 o;
            o.x = __builtin_amdgcn_perm(xv[t].z, xv[t].x, 0x05040100u);   // (x0, x4)
            o.y = __builtin_amdgcn_perm(xv[t].z, xv[t].x, 0x07060302u);   // (x1, x5)
            o.z = __builtin_amdgcn_perm(xv[t].w, xv[t].y, 0x05040100u);   // (x2, x6)
            o.w = __builtin_amdgcn_perm(xv[t].w, xv[t].y, 0x07060302u);   // (x3, x7)
            L.xs[m * WS + g * 8u + t] = o;
            s0 = dot2_bf16(xv[t].x, kOnePair, s0);
            s1 = dot2_bf16(xv[t].y, kOnePair, s1);
            s0 = dot2_bf16(xv[t].z, kOnePair, s0);
            s1 = dot2_bf16(xv[t].w, kOnePair, s1);
        }
        reinterpret_cast<float*>(L.sx)[g * 4u + m] = s0 + s1;
    }
    for (uint32_t t = tid; t < WS; t += kThreads) L.zs[t] = uint4{0u, 0u, 0u, 0u};
    __syncthreads();
}

// The per-wave constants of one op: this wave's split and its range of group pairs.
struct WaveRange {
    uint32_t tid, lane, wave, split, sh, S, j, kb, pairs, first, cnt, last;
};

__device__ __forceinline__ WaveRange wave_range(ConstStepOp& d, uint32_t tid) {
    WaveRange r;
    r.tid = tid;
    r.lane = tid & 63u;
    r.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    r.S = d.splits;
    r.sh = d.split_shift;
    r.split = r.wave & (r.S - 1u);
    r.j = r.lane & 15u;
    r.kb = r.lane >> 4;
    r.pairs = d.pairs;
    const uint32_t per = r.pairs >> r.sh;
    const uint32_t rem = r.pairs & (r.S - 1u);
    r.first = r.split * per + min(r.split, rem);
    r.cnt = per + (r.split < rem ? 1u : 0u);
    r.last = r.first + r.cnt - 1u;
    return r;
}

// One wave's part of one 16-wave block: its loaded weights and where its rows go.
struct BlockLoads {
    Batch<4> ba, bb;
    uint32_t sbl[1][4];
    uint16_t* y;
    uint32_t n;
    uint32_t tile;
    uint32_t gtile;
    LaneMatrix lm;
};

// Issue this wave's weight loads of block vb (16 / S row tiles, S waves per tile, as one
// workgroup of the per-call kernel); with first_only, only the scales and the first batch
// of four pairs (the second batch is issued by the caller). A plain op's segment is read by index, so only its
// fields are live; a gate/up op alternates gate and up tiles (virtual tile 2t is gate
// tile t, 2t + 1 up tile t).
__device__ __forceinline__ void issue_block(ConstStepOp& d, bool dual, uint32_t vb, const WaveRange& r,
                                            BlockLoads& bl, bool first_only) {
    const uint32_t gtile = (vb << (4u - r.sh)) + (r.wave >> r.sh);
    const uint4* codes;
    const uint2* sb;
    if (dual) {
        codes = (gtile & 1u) ? d.codes2 : d.seg[0].codes;
        sb = (gtile & 1u) ? d.sb2 : d.seg[0].sb;
        bl.y = d.seg[0].y;
        bl.n = d.seg[0].n;
        bl.tile = gtile >> 1;
    } else {
        const uint32_t nseg = d.nseg;
        const uint32_t si = (nseg > 1u && gtile >= d.seg[1].tile_begin ? 1u : 0u) +
                            (nseg > 2u && gtile >= d.seg[2].tile_begin ? 1u : 0u);
        const __attribute__((address_space(4))) StepSegment& sg = d.seg[si];
        codes = sg.codes;
        sb = sg.sb;
        bl.y = sg.y;
        bl.n = sg.n;
        bl.tile = gtile - sg.tile_begin;
    }
    bl.gtile = gtile;
    const uint32_t tiles = (bl.n + kTileRows - 1u) / kTileRows;
    const uint32_t ltile = min(bl.tile, tiles - 1u);   // tiles past the matrix are loaded, never stored
    LaneMatrix lm;
    lm.codes = buffer_rsrc(codes, tiles * r.pairs * 1024u);
    lm.sb = buffer_rsrc(sb, tiles * r.pairs * 128u);
    lm.c_off = (ltile * r.pairs * 64u + r.lane) * 16u;
    lm.sb_off = (ltile * r.pairs * 16u + r.j) * 8u;
    const uint32_t ob = r.kb;
    const uint32_t off = (ltile * r.pairs * 16u + (ob >> 1) * 16u + r.j) * 8u + (ob & 1u) * 4u;
#pragma unroll
    for (int b = 0; b < 4; ++b)
        bl.sbl[0][b] = __builtin_amdgcn_raw_buffer_load_b32(lm.sb, off, (r.first + 2u * b) * 128u, kStreamPolicy);
    load_batch<4, false>(lm, r.first, r.last, bl.ba);
    if (!first_only) load_batch<4, false>(lm, r.first + 4u, r.last, bl.bb);
    bl.lm = lm;
}

// Compute a block's loads against the staged x, reduce the splits and store the rows
// (coherently: later ops of the launch read them on other compute units). A gate/up op's
// gate tiles take the matching up rows from LDS for the GELU epilogue.
template <int M>
__device__ __forceinline__ void finish_block(const BlockLoads& bl, bool dual, const OpLds& L, uint32_t G,
                                             uint32_t WS, const WaveRange& r) {
    // Opaque VGPR values, so (w & mask) | bits selects v_and_or_b32 (see and_or).
    uint32_t mask = kNibbleMask;
    uint32_t bits = kMagic128;
    asm volatile("" : "+v"(mask), "+v"(bits));
    float y[1][M];
#pragma unroll
    for (int m = 0; m < M; ++m) y[0][m] = 0.0f;
    const Batch<4> ba[1] = {bl.ba};
    const Batch<4> bb[1] = {bl.bb};
    compute_lane_groups<M, 1, 4>(ba, bb, bl.sbl, r.first, r.cnt, G, L.xs, L.zs, WS, L.sx, r.lane, mask, bits, y);
    reduce_splits<M, 1>(y, L.red, r.wave, r.split, r.S, r.kb, r.j);
    const uint32_t out_row = bl.tile * kTileRows + r.j;
    const bool writer = r.split == 0u && r.kb == 0u;
    float* cs = L.comb + ((r.wave >> r.sh) >> 1) * M * kTileRows;
    if (dual) {
        if (writer && (bl.gtile & 1u)) {
#pragma unroll
            for (int m = 0; m < M; ++m) cs[m * kTileRows + r.j] = round_bf16(y[0][m]);
        }
        __syncthreads();
    }
    if (writer && out_row < bl.n && !(dual && (bl.gtile & 1u))) {
        const __amdgpu_buffer_rsrc_t yr = buffer_rsrc(bl.y, M * bl.n * 2u);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float out = dual ? gate_up_value(y[0][m], cs[m * kTileRows + r.j]) : round_bf16(y[0][m]);
            __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(out), yr, (m * bl.n + out_row) * 2u, 0, kCoherent);
        }
    }
}

// One op for this workgroup: its blocks vb = blockIdx.x, + gridDim.x, ... The first
// block's weight loads are issued before the wait for op - 1.
template <int M>
__device__ __forceinline__ bool run_op(ConstStepOp& d, uint32_t op, uint32_t* sync, uint32_t target,
                                       uint32_t spin_limit, uint4* smem) {
    const uint32_t k = d.k;
    const uint32_t G = k / 64u;
    const uint32_t WS = k / 8u + 1u;
    const bool norm = d.form == static_cast<uint32_t>(StepForm::kNorm);
    const bool dual = d.form == static_cast<uint32_t>(StepForm::kDual);
    const OpLds L = op_lds<M>(smem, WS, G, norm);
    // The thread index, opaque per op: the compiler would otherwise hoist every lane
    // predicate derived from it out of the op loop and keep them all live (spilling).
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const WaveRange r = wave_range(d, tid);
    const uint32_t vbs = d.vbs;

    BlockLoads bl;
    const bool have = blockIdx.x < vbs;   // workgroup-uniform
    // The first batch goes out before the wait and the second after x is staged: every
    // later vector-memory request of the compute unit (the polls, the x loads) queues behind
    // the loads already issued, so a deeper prefetch delays the op's start.
    if (op > 0u) arrive(sync, op - 1u, r.tid);
    if (have) issue_block(d, dual, blockIdx.x, r, bl, true);
    if (op > 0u && !wait_all(sync, op - 1u, target, spin_limit, L.ctl, r.lane, r.wave)) return false;
    if (!have) return true;
    stage_x<M>(d, L, norm, k, G, WS, r.tid, r.lane, r.wave);
    load_batch<4, false>(bl.lm, r.first + 4u, r.last, bl.bb);
    finish_block<M>(bl, dual, L, G, WS, r);
    for (uint32_t vb = blockIdx.x + gridDim.x; vb < vbs; vb += gridDim.x) {
        issue_block(d, dual, vb, r, bl, false);
        __syncthreads();   // the previous block's reduction and combine areas have been read
        finish_block<M>(bl, dual, L, G, WS, r);
    }
    // The storing waves' outputs are complete before this workgroup arrives for the op.
    if (r.split == 0u) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return true;
}

template <int M>
__global__ __launch_bounds__(kThreads) void q4_step_program_kernel(ConstStepOp* ops, uint32_t n_ops, uint32_t* sync,
                                                                  uint32_t spin_limit) {
    extern __shared__ __attribute__((aligned(16))) uint4 smem[];
    const uint32_t epoch = __builtin_amdgcn_readfirstlane(sys_load(sync + kSyncEpoch));
    const uint32_t target = (epoch + 1u) * (gridDim.x / kStepSlots);
    for (uint32_t i = 0; i < n_ops; ++i) {
        const bool ok = run_op<M>(ops[i], i, sync, target, spin_limit, smem);
        if (!ok) return;
    }
    // Count this workgroup finished; the last one of the run advances the epoch, which the
    // next run reads at its start (the launch boundary orders the two).
    __syncthreads();
    if (threadIdx.x == 0u) {
        const uint32_t prev = __hip_atomic_fetch_add(sync + kSyncDone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        if (prev + 1u == (epoch + 1u) * gridDim.x)
            __hip_atomic_store(sync + kSyncEpoch, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

using StepKernel = void (*)(ConstStepOp*, uint32_t, uint32_t*, uint32_t);

StepKernel step_kernel(uint32_t m) {
    switch (m) {
        case 1: return q4_step_program_kernel<1>;
        case 2: return q4_step_program_kernel<2>;
        case 3: return q4_step_program_kernel<3>;
        case 4: return q4_step_program_kernel<4>;
        default: throw NativeError(HYP_STATUS_INTERNAL, "step program: m outside 1..4");
    }
}

// Allow the kernel the device's whole LDS per workgroup (once per device and m).
void configure(StepKernel kernel, uint32_t m) {
    static thread_local int configured[kSkinnyMaxM + 1] = {-1, -1, -1, -1, -1};
    int dev = 0;
    HYP_HIP_CHECK(hipGetDevice(&dev));
    if (configured[m] != dev) {
        int lds = 0;
        HYP_HIP_CHECK(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
        HYP_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, lds));
        configured[m] = dev;
    }
}

}  // namespace

size_t step_op_lds_bytes(uint32_t m, uint32_t k, StepForm form) {
    const size_t W = k / 8u;
    const size_t G = k / 64u;
    const bool dual = form == StepForm::kDual;
    const bool norm = form == StepForm::kNorm;
    return 16u + (m + 1u) * (W + 1u) * 16u + G * 16u + static_cast<size_t>(kStepWaves) * m * kTileRows * 4u +
           (norm ? (m * G + m) * 4u : 0u) + (dual ? static_cast<size_t>(kStepWaves / 2u) * m * kTileRows * 4u : 0u);
}

uint32_t step_program_grid(uint32_t m, size_t lds) {
    const StepKernel kernel = step_kernel(m);
    configure(kernel, m);
    int per_cu = 0;
    HYP_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kernel),
                                                               static_cast<int>(kThreads), lds));
    HYP_REQUIRE(per_cu >= 1, HYP_STATUS_UNSUPPORTED, "step program: a 16-wave workgroup does not fit a compute unit");
    const uint32_t cus = device_compute_units();
    const uint32_t grid = cus / kStepSlots * kStepSlots;
    HYP_REQUIRE(grid >= kStepSlots, HYP_STATUS_UNSUPPORTED, "step program: too few compute units");
    return grid;
}

void launch_step_program(const StepOp* d_ops, uint32_t n_ops, uint32_t m, uint32_t* d_sync, uint32_t grid,
                         size_t lds, uint32_t spin_limit, hipStream_t stream) {
    const StepKernel kernel = step_kernel(m);
    configure(kernel, m);
    ConstStepOp* ops = reinterpret_cast<ConstStepOp*>(reinterpret_cast<uintptr_t>(d_ops));
    void* args[] = {&ops, &n_ops, &d_sync, &spin_limit};
    HYP_HIP_CHECK(hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kernel), dim3(grid), dim3(kThreads), args,
                                             static_cast<unsigned int>(lds), stream));
}

}  // namespace hyperion::hip
