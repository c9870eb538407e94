// Host side of the decode-step program (step_program.h): validation of the ops, the
// per-op k split (the per-call entry points' choice, so results match them bit for bit),
// the device copies of the op descriptors and the synchronisation words, and the launch.
#include "step_program_host.h"

#include <algorithm>
#include <string>

#include "q4_layout.h"

namespace hyperion::model {

using hip::NativeError;
using hip::StepForm;
using hip::StepOp;

namespace {

constexpr uint32_t kDefaultSpinLimit = 1u << 21;   // ~2 s of polling before a run gives up
constexpr uint32_t kMaxPairsPerWave = 8u;           // two register batches of 4 pairs

std::string op_name(size_t i) { return "step program op " + std::to_string(i) + ": "; }

}  // namespace

StepProgram::StepProgram(const std::vector<StepOpSpec>& specs, uint32_t m, uint32_t spin_limit)
    : m_(m), n_ops_(static_cast<uint32_t>(specs.size())),
      spin_limit_(spin_limit == 0u ? kDefaultSpinLimit : spin_limit) {
    HYP_REQUIRE(m >= 1u && m <= hip::kSkinnyMaxM, HYP_STATUS_INVALID_ARGUMENT, "step program: m must be 1..4");
    HYP_REQUIRE(!specs.empty(), HYP_STATUS_INVALID_ARGUMENT, "step program: no ops");
    std::vector<StepOp> ops(specs.size());
    size_t lds = 0;
    int dev = 0;
    HYP_HIP_CHECK(hipGetDevice(&dev));
    int max_lds = 0;
    HYP_HIP_CHECK(hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    for (size_t i = 0; i < specs.size(); ++i) {
        const StepOpSpec& s = specs[i];
        StepOp& d = ops[i];
        d = StepOp{};
        const std::string who = op_name(i);
        HYP_REQUIRE(s.x != nullptr, HYP_STATUS_INVALID_ARGUMENT, who + "x must be a non-null device pointer");
        const bool dual = s.form == StepForm::kDual;
        HYP_REQUIRE(dual ? s.count == 2u : (s.count >= 1u && s.count <= hip::kStepMaxSegments),
                    HYP_STATUS_INVALID_ARGUMENT, who + (dual ? "gate/up takes exactly two weights" : "count must be 1..3"));
        const uint32_t k = s.w[0]->mat.k;
        uint32_t tiles_total = 0;
        const uint32_t nseg = dual ? 1u : s.count;
        for (uint32_t q = 0; q < s.count; ++q) {
            const hip::Q4Matrix& w = s.w[q]->mat;
            HYP_REQUIRE(w.k == k, HYP_STATUS_INVALID_ARGUMENT, who + "the op's weights must share k");
            HYP_REQUIRE(w.codes != nullptr && w.sb != nullptr, HYP_STATUS_INTERNAL,
                        who + "weights are not in the tiled resident layout");
            HYP_REQUIRE(hip::TiledDims::of(w.n, w.k).code_bytes() < (1ull << 31), HYP_STATUS_UNSUPPORTED,
                        who + "a matrix exceeds 2 GiB of packed codes");
        }
        if (dual) {
            HYP_REQUIRE(s.w[1]->mat.n == s.w[0]->mat.n, HYP_STATUS_INVALID_ARGUMENT,
                        who + "gate and up must have the same shape");
            HYP_REQUIRE(s.y[0] != nullptr, HYP_STATUS_INVALID_ARGUMENT, who + "y[0] must be a non-null device pointer");
        }
        for (uint32_t q = 0; q < nseg; ++q) {
            const hip::Q4Matrix& w = s.w[q]->mat;
            HYP_REQUIRE(s.y[q] != nullptr, HYP_STATUS_INVALID_ARGUMENT, who + "y[i] must be non-null device pointers");
            d.seg[q] = hip::StepSegment{w.codes, w.sb, s.y[q], w.n, tiles_total};
            tiles_total += hip::TiledDims::of(w.n, w.k).tiles;
        }
        if (dual) tiles_total *= 2u;   // gate and up tiles alternate
        const uint32_t pairs = hip::TiledDims::of(16u, k).pairs;
        const uint32_t splits = hip::choose_skinny_splits(
            tiles_total, pairs, m, dual ? hip::SkinnyForm::kDual : hip::SkinnyForm::kPlain);
        const uint32_t per_wave = (pairs + splits - 1u) / splits;
        HYP_REQUIRE(per_wave <= kMaxPairsPerWave, HYP_STATUS_UNSUPPORTED,
                    who + "k = " + std::to_string(k) + " leaves " + std::to_string(per_wave) +
                        " group pairs per wave, more than one launch holds in registers");
        HYP_REQUIRE(splits >= 1u && splits <= (dual ? 4u : hip::kStepWaves) && pairs >= splits,
                    HYP_STATUS_INTERNAL, who + "bad split");
        if (s.form == StepForm::kNorm) {
            HYP_REQUIRE(std::isfinite(s.eps) && s.eps >= 0.0f, HYP_STATUS_INVALID_ARGUMENT,
                        who + "eps must be finite and >= 0");
        }
        d.x = s.x;
        d.codes2 = dual ? s.w[1]->mat.codes : nullptr;
        d.sb2 = dual ? s.w[1]->mat.sb : nullptr;
        d.form = static_cast<uint32_t>(s.form);
        d.nseg = nseg;
        d.k = k;
        d.pairs = pairs;
        d.splits = splits;
        d.split_shift = static_cast<uint32_t>(__builtin_ctz(splits));
        const uint32_t tiles_per_block = hip::kStepWaves / splits;
        d.vbs = (tiles_total + tiles_per_block - 1u) / tiles_per_block;
        d.eps = s.form == StepForm::kNorm ? s.eps : 0.0f;
        d.norm_w = s.form == StepForm::kNorm ? s.norm_w : nullptr;
        const size_t op_lds = hip::step_op_lds_bytes(m, k, s.form);
        HYP_REQUIRE(op_lds <= static_cast<size_t>(max_lds), HYP_STATUS_UNSUPPORTED,
                    who + "x of " + std::to_string(m) + " x " + std::to_string(k) + " exceeds the LDS");
        lds = std::max(lds, op_lds);
    }
    lds_ = lds;
    grid_ = hip::step_program_grid(m, lds_);
    ops_ = DeviceBuffer(ops.size() * sizeof(StepOp));
    HYP_HIP_CHECK(hipMemcpy(ops_.data(), ops.data(), ops.size() * sizeof(StepOp), hipMemcpyHostToDevice));
    sync_ = DeviceBuffer(static_cast<size_t>(hip::sync_words(n_ops_)) * sizeof(uint32_t));
    reset();
}

void StepProgram::reset() {
    HYP_HIP_CHECK(hipMemset(sync_.data(), 0, sync_.bytes()));
    HYP_HIP_CHECK(hipDeviceSynchronize());
}

void StepProgram::run(hipStream_t stream) const {
    hip::launch_step_program(static_cast<const StepOp*>(ops_.data()), n_ops_, m_,
                             static_cast<uint32_t*>(sync_.data()), grid_, lds_, spin_limit_, stream);
}

uint32_t StepProgram::check() {
    HYP_HIP_CHECK(hipDeviceSynchronize());
    uint32_t err = 0;
    HYP_HIP_CHECK(hipMemcpy(&err, static_cast<uint32_t*>(sync_.data()) + hip::kSyncError, sizeof(err),
                            hipMemcpyDeviceToHost));
    if (err != 0u) reset();
    return err;
}

}  // namespace hyperion::model
