// Host object of a decode-step program (step_program.h).
#pragma once

#include <cmath>
#include <cstdint>
#include <vector>

#include "qlinear.h"
#include "step_program.h"

namespace hyperion::model {

// One op as the caller describes it: weights are resident projections; x and y device
// pointers that stay valid while the program is used.
struct StepOpSpec {
    hip::StepForm form = hip::StepForm::kPlain;
    uint32_t count = 0;                         // weights used (dual: gate, up)
    const QuantizedLinear* w[hip::kStepMaxSegments] = {};
    const uint16_t* x = nullptr;
    uint16_t* y[hip::kStepMaxSegments] = {};
    float eps = 0.0f;
    const uint16_t* norm_w = nullptr;           // kNorm: the norm's bf16 weight [k], or null
};

class StepProgram {
  public:
    // Validates every op and copies the descriptors to the device. spin_limit 0 = default.
    StepProgram(const std::vector<StepOpSpec>& ops, uint32_t m, uint32_t spin_limit);
    // Enqueue one run (one cooperative launch) on stream.
    void run(hipStream_t stream) const;
    // Wait for the device, then return the error word of the runs so far (0: none) and,
    // if set, clear the synchronisation words so the program can run again.
    uint32_t check();

    [[nodiscard]] uint32_t grid() const noexcept { return grid_; }

  private:
    void reset();

    uint32_t m_;
    uint32_t n_ops_;
    uint32_t spin_limit_;
    uint32_t grid_ = 0;
    size_t lds_ = 0;
    DeviceBuffer ops_;
    DeviceBuffer sync_;
};

}  // namespace hyperion::model
