// The mlp_stack glue shared by the C ABI's stack entry points (internal): argument checks, the scratch layout of one
// call and the call itself on a given scratch base.
#pragma once

#include "common.hpp"
#include "gemm_kernels.hpp"

namespace sepal::hip {

// Throws InvalidArgument for a kind, shape, act_block or pointer sepal_hip_mlp_stack refuses.
void check_stack_args(int32_t kind, std::size_t hidden, std::size_t inter, const void* x, const int8_t* const* w_gate_up,
                      const float* const* s_gate_up, const int8_t* const* w_down, const float* const* s_down, const float* y,
                      std::size_t act_block);

// Where an mlp_stack call keeps its scratch, as offsets from the scratch base (the split-K zone of the small-M
// multiplies first, [0, kScratchOffset)); `end` is the bytes it needs.
struct StackZones {
    enum Form { SMALL_W8G, SMALL_Q8, GENERAL } form = GENERAL;
    SmallStackPlan plan{};
    bool per_token = false, fused_h = false;
    std::size_t ab_h = 128, ab_i = 128;
    std::size_t off_h = 0, off_p = 0;                                          // H, the small forms' K-part sums
    std::size_t off_hmax = 0, off_qx = 0, off_sx = 0, off_qh = 0, off_sh = 0;  // q8: int8 operands and scales
    std::size_t off_split = 0;                                                 // kind 2: the hi + lo pairs of H
    // w8g at large M: the widened weight images of the gate/up and down weights (0 bytes: the kernels widen)
    std::size_t off_img = 0, img = 0, off_img_dn = 0, img_dn = 0;
    std::size_t end = 0;
};

StackZones stack_zones(int kind, std::size_t t, std::size_t hidden, std::size_t inter, std::size_t act_block);

// One call of the stack on the scratch at `ws` (laid out by stack_zones; its counter zone zero at rest). img_gate_up /
// img_down (null, or one load-time weight image per layer): the w8g multiplies read them instead of widening the
// weights into the workspace's images (z.img and z.img_dn are then 0). stream_w: the M <= 16 forms' weights (w8g and
// q8) are in the stream layout (launch_stream_layout).
void run_stack(const StackZones& z, int kind, std::size_t layers, std::size_t t, std::size_t hidden, std::size_t inter,
               void* x, const int8_t* const* w_gate_up, const float* const* s_gate_up, const int8_t* const* w_down,
               const float* const* s_down, float* y, double eps, char* ws, hipStream_t st,
               const void* const* img_gate_up = nullptr, const void* const* img_down = nullptr, bool stream_w = false);

} // namespace sepal::hip
