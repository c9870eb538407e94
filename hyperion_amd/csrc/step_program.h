// A decode-step program: an ordered list of skinny (m <= 4) quantized-matmul ops that one
// persistent launch runs back to back (q4_step_program.hip). Shared by the host builder
// (step_program.cc) and the kernel.
//
// Every op reads its input x as written by earlier ops of the same launch (or before the
// launch) and writes its outputs y; op i starts only after every workgroup has finished op
// i - 1 (arrival counters in device memory), so an op may read what any earlier op wrote
// and overwrite what any earlier op read. Results are the bits the per-call entry points
// give with the same k splits: the same device functions do the arithmetic.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace hyperion::hip {

constexpr uint32_t kStepWaves = 16;       // waves per workgroup (one workgroup per compute unit)
constexpr uint32_t kStepSlots = 8;        // arrival counters per op; workgroup w counts in slot w % 8
constexpr uint32_t kStepMaxSegments = 3;  // projections sharing x in one op (q, k, v)

enum class StepForm : uint32_t {
    kPlain = 0,   // ys[i] = x . W_i^T for the op's segments
    kNorm = 1,    // the same on rms-normalised x rows (the normalised rows are not written)
    kDual = 2,    // y = bf16(gelu_tanh(x . G^T) * (x . U^T)), one segment
};

struct StepSegment {
    const uint4* codes;   // tiled layout (q4_layout.h)
    const uint2* sb;
    uint16_t* y;          // [m, n]
    uint32_t n;
    uint32_t tile_begin;  // first 16-row tile of this segment among the op's tiles
};

struct StepOp {
    const uint16_t* x;    // [m, k] bf16
    const uint4* codes2;  // kDual: the up projection (same n, k as segment 0)
    const uint2* sb2;
    StepSegment seg[kStepMaxSegments];
    uint32_t form;        // StepForm
    uint32_t nseg;
    uint32_t k;
    uint32_t pairs;       // ceil(k / 128)
    uint32_t splits;      // waves sharing a 16-row tile (power of two, <= 16)
    uint32_t split_shift;
    uint32_t vbs;         // 16-wave blocks of 16 / splits tiles each
    float eps;            // kNorm
    uint32_t pad;
    const uint16_t* norm_w;   // kNorm: the norm's bf16 weight [k], or null
};

// Device synchronisation words of one program (uint32 indices; each on its own 128-byte
// line): the run count, the workgroups finished over all runs, an error flag, and then
// kStepSlots arrival counters per op.
constexpr uint32_t kSyncEpoch = 0;
constexpr uint32_t kSyncDone = 32;
constexpr uint32_t kSyncError = 64;
constexpr uint32_t kSyncCounters = 96;
constexpr uint32_t kSyncStride = 32;      // words between two counters
constexpr uint32_t sync_words(uint32_t n_ops) { return kSyncCounters + n_ops * kStepSlots * kSyncStride; }

// Error codes left in the error word by a run that gave up waiting.
constexpr uint32_t kStepErrTimeout = 1;   // a workgroup waited past the spin limit

// Dynamic LDS of the program kernel at m rows for an op of k columns.
size_t step_op_lds_bytes(uint32_t m, uint32_t k, StepForm form);
// Launch one run: `grid` workgroups (a multiple of kStepSlots, all co-resident: a
// cooperative launch), `lds` bytes of dynamic LDS (the maximum over the ops).
void launch_step_program(const StepOp* d_ops, uint32_t n_ops, uint32_t m, uint32_t* d_sync, uint32_t grid,
                         size_t lds, uint32_t spin_limit, hipStream_t stream);
// Workgroups the program kernel runs with: one per compute unit, rounded down to a
// multiple of kStepSlots, after checking that one workgroup fits per compute unit.
uint32_t step_program_grid(uint32_t m, size_t lds);

}  // namespace hyperion::hip
