// Launchers of the HIP kernels (internal). The C ABI (capi.cpp) validates the arguments and calls these.
#pragma once

#include "common.hpp"

namespace sepal::hip {

// Rows at or below which the multiplies take the weight-streaming small-M path.
inline constexpr std::size_t kSmallM = 64;

// Default routing of the q8 multiply (config -1): the small-M (streaming) kernels up to kSmallM rows, except above 32
// rows with N >= 8192, where the large-M kernels are faster (gate/up 19456 x 2560 at T = 40-64: 28-30 against 41-43 us
// per token, 35-37 against 43-44 per 128; 12288 x 2560: 29-33 against 35) and also bit-exact to cpu-q8.
inline bool q8_streams(std::size_t t, std::size_t n) { return t <= kSmallM && (t <= 32 || n < 8192); }

struct GemmArgs {
    const void* x = nullptr;
    int x_type = SEPAL_HIP_BF16;
    std::size_t ld_x = 0;
    const std::int8_t* w = nullptr;
    std::size_t ld_w = 0;
    const float* s = nullptr;
    std::size_t ld_s = 0;
    void* y = nullptr;
    int y_type = SEPAL_HIP_F32;
    std::size_t ld_y = 0;
    std::size_t t = 0, n = 0, k = 0;
    int epilogue = SEPAL_HIP_STORE;
    int config = -1;
    int force_splits = 0;  // small-M: > 0 forces the number of K splits (tests)
    bool w_stream = false;  // M <= 16 pass kernels only: w in the stream layout (launch_stream_layout; ld_w unused)
    // q8 only
    const float* xs = nullptr;
    std::size_t ld_xs = 0;
    std::size_t act_block = 128;
    std::int32_t* sums = nullptr;  // group-sum mode
    float* ys = nullptr;           // kSwigluQ8: output scales [t, ld_ys], one per 128 columns of y
    std::size_t ld_ys = 0;
    // scratch the caller (the C ABI) carves out of its workspace:
    void* scratch = nullptr;  // the zero-at-rest split-K counters (kCounterBytes) followed by kPartialBytes of partials
    void* xsplit = nullptr;   // w8g with float32 X: the bf16 hi + lo pairs
    float* ytmp = nullptr;    // w8g with float32 X and SwiGLU off the one-pass kernel: the float32 sums [t, n]
    void* wimage = nullptr;   // w8g at large M: room for the widened weight image (gemm_w8g_image_bytes)
    std::size_t wimage_bytes = 0;
    bool image_ready = false;  // the image already holds these weights (widened by the previous multiply of a stack)
    // w8g at large M in a stack: the next multiply's weights, widened into next_image by the spare blocks of this
    // multiply's last launch (or by a launch of its own after it); next_f16: widen to binary16, else bf16
    const std::int8_t* next_w = nullptr;
    std::size_t next_ld_w = 0, next_n = 0, next_k = 0;
    int next_f16 = 0;
    void* next_image = nullptr;
};

// q8 epilogue (internal, not in the public enum): SwiGLU, then the output quantized to int8 per row and 128 columns
// (rule RECIPROCAL); y is int8 [t, ld_y], the scales go to ys.
constexpr int kSwigluQ8 = 16;

void launch_gemm_w8g(const GemmArgs& a, hipStream_t stream);
// w8g Y type (internal, not in the public enum): the SwiGLU output as bf16 hi + lo pairs in the row layout the float32-X
// down multiply reads (y [t, 2 ld_y] bf16), the split of the float32 value as that multiply's own split pass makes it.
constexpr int kYPairs = 17;
// Whether a stack's gate/up multiply `gu` (SwiGLU) can write its H as kYPairs for the down multiply `dn` (float32 X):
// both run on the large-M kernels, the down multiply on its one-pass hi + lo form.
bool gemm_w8g_pairs_chain(const GemmArgs& gu, const GemmArgs& dn);
// The down multiply of such a chain: dn.x holds the pairs (bf16 [t, 2 dn.k], row stride dn.ld_x values).
void launch_gemm_w8g_pairs(const GemmArgs& dn, hipStream_t stream);
// Scratch bytes launch_gemm_w8g needs at xsplit (then ytmp, 256-byte aligned, when non-zero) for this problem; 0 for a
// 16-bit X.
std::size_t gemm_w8g_scratch_bytes(const GemmArgs& a);
// Bytes of the widened weight image the large-M w8g kernels use for this problem (0: they widen in the kernel). The
// image is written by every call, so it only needs to be scratch.
std::size_t gemm_w8g_image_bytes(const GemmArgs& a);
// The weight image as a load-time form: its bytes for an N x K matrix (0 when its offsets would exceed 32 bits) and
// the widening pass (binary16 when f16, else bf16) into `img`.
std::size_t w8g_image_bytes_nk(std::size_t n, std::size_t k);
void launch_w8g_image(const std::int8_t* w, std::size_t ld_w, std::size_t n, std::size_t k, bool f16, void* img,
                      hipStream_t stream);
// The part of gemm_w8g_scratch_bytes that is the split buffer (ytmp follows it).
inline std::size_t gemm_w8g_split_bytes(const GemmArgs& a) { return (a.t * a.k * 4 + 255) / 256 * 256; }
void launch_stream_w8g(const GemmArgs& a, hipStream_t stream);
void launch_stream_q8(const GemmArgs& a, hipStream_t stream);
void launch_gemm_q8(const GemmArgs& a, hipStream_t stream);
// The int8-activation multiply with per-channel weight scales: y = (float(sum over K of xq * wq) * xs[t]) * s[n] (a.s
// holds one scale per row, a.ld_s = 1); y float32 or binary16 (a.y_type).
void launch_gemm_s8(const GemmArgs& a, hipStream_t stream);
void launch_gemm_q8y(const GemmArgs& a, hipStream_t stream);
// The GPU int8 path's per-row quantizer (rule 127 / amax, zero rows scale 0), with an optional per-column factor.
void launch_s8_quantize_rows(const void* x, int x_type, std::size_t ld_x, const float* smooth, std::int8_t* q, std::size_t ld_q,
                             float* scales, std::size_t rows, std::size_t cols, hipStream_t stream);
void launch_broadcast_scales(const float* sw, float* s, std::size_t n, std::size_t groups, hipStream_t stream);
// Column statistics of binary16 x: sums null -> amax[c] = max |x[:, c]|; else amax[c] = max(amax[c], ...), sums[c] +=
// sum |x|, sums[cols + c] += sum x^2 (double, rows in order).
void launch_column_stats(const void* x, std::size_t ld_x, std::size_t rows, std::size_t cols, float* amax, double* sums,
                         hipStream_t stream);
void launch_f32_to_f16(const float* src, std::size_t ld_src, std::uint16_t* dst, std::size_t ld_dst, std::size_t rows,
                       std::size_t cols, hipStream_t stream);
void launch_q8_group_sums(const GemmArgs& a, hipStream_t stream);
void launch_gemm_q8_swiglu_q8(const GemmArgs& a, hipStream_t stream);  // large-M kernel only

void launch_quantize_group(const void* src, int src_type, std::size_t ld_src, const void* src_up, std::int8_t* q,
                           std::size_t ld_q, float* s, std::size_t ld_s, std::size_t rows, std::size_t k, int rule,
                           std::size_t inter, hipStream_t stream);
void launch_quantize_rows(const void* x, int x_type, std::size_t ld_x, std::int8_t* q, std::size_t ld_q, float* scales,
                          std::size_t ld_s, std::size_t rows, std::size_t cols, std::size_t block, hipStream_t stream);
void launch_rmsnorm(const float* x, std::size_t ld_x, void* y, int y_type, std::size_t ld_y, const float* w1,
                    std::size_t rows, std::size_t cols, double eps, hipStream_t stream);
void launch_rmsnorm_quantize(const float* x, std::size_t ld_x, std::uint16_t* y_bf16, std::size_t ld_y, const float* w1,
                             std::int8_t* q, std::size_t ld_q, float* scales, std::size_t ld_s, std::size_t rows,
                             std::size_t cols, std::size_t block, double eps, hipStream_t stream);
void launch_f32_to_bf16(const float* src, std::uint16_t* dst, std::size_t count, hipStream_t stream);

// Edge shapes (edge.hip): a zero-padded copy of `rows` rows of `bytes` bytes (src may be null when bytes is 0) into rows
// of ld_dst_bytes (a multiple of 4); and y[:, 0:cols] = tmp (or += tmp for add; y float32 or binary16, rounded).
void launch_pad_rows(const void* src, std::size_t ld_src_bytes, void* dst, std::size_t ld_dst_bytes, std::size_t rows,
                     std::size_t bytes, hipStream_t stream);
void launch_put_cols(const float* tmp, std::size_t ld_tmp, void* y, int y_type, std::size_t ld_y, std::size_t rows,
                     std::size_t cols, bool add, hipStream_t stream);

// Packed-weight files (packed_file.hip): the device fingerprint of a byte range (`lanes` holds
// fingerprint_scratch_bytes()), and the synchronous save / load of one packed matrix.
void launch_fingerprint(const void* data, std::size_t bytes, std::uint64_t* out, void* lanes, hipStream_t stream);
std::size_t fingerprint_scratch_bytes();
void packed_save(const char* path, const std::int8_t* q, std::size_t ld_q, const float* s, std::size_t ld_s,
                 std::size_t rows, std::size_t k, int rule, int layout, std::uint64_t source_fp, void* scratch,
                 hipStream_t stream);
void packed_load(const char* path, std::int8_t* q, std::size_t ld_q, float* s, std::size_t ld_s, std::size_t rows,
                 std::size_t k, int rule, int layout, std::uint64_t source_fp, void* scratch, hipStream_t stream);

// The M <= 16 w8g layer of the MLP stack (stack_small.hip): a launch plan for one shape and device, and one layer.
struct SmallStackPlan {
    int blocks;           // blocks of the gate/up pass grid (one per CU)
    int tiles_per_block;  // gate/up weight tiles (8 features) per block
    int parts;            // K-parts of the down pass
    int units_per_block;  // (K-part, column tile) units per block of the down pass
};
bool small_stack_plan(std::size_t t, std::size_t hidden, std::size_t inter, SmallStackPlan& plan);
// One w8g multiply at T <= 16 on the stack's pass kernels: SwiGLU straight to Y, Store / Add through K-parts in the
// workspace's partial zone and a parts sum. small_gemm_plan returns false for shapes the pass kernels do not take.
struct SmallGemmPlan {
    int parts;      // K-parts (1 for SwiGLU)
    int per_block;  // weight tiles (SwiGLU) or (K-part, column tile) units per block
    std::size_t lds;
};
bool small_gemm_plan(const GemmArgs& a, SmallGemmPlan& plan);
void launch_small_gemm_w8g(const GemmArgs& a, const SmallGemmPlan& plan, hipStream_t stream);
// The q8 form for the SwiGLU multiply (float32 H): the gate/up pass of the q8 stack.
bool small_gemm_plan_q8(const GemmArgs& a, SmallGemmPlan& plan);
void launch_small_gemm_q8(const GemmArgs& a, const SmallGemmPlan& plan, hipStream_t stream);
// The exact int32 group sums (a.sums [K/128][T][N]) from the pass kernels' int8 MFMAs at T <= 16 (the gate/up pass
// when N is a multiple of 128, else the K-parts pass); false when no pass plan takes the shape.
bool small_q8_group_sums(const GemmArgs& a, hipStream_t stream);
// ... and for the Store / Add multiply (float32 Y through K-parts and the parts sum).
bool small_gemm_plan_q8_parts(const GemmArgs& a, SmallGemmPlan& plan);
void launch_small_gemm_q8_parts(const GemmArgs& a, const SmallGemmPlan& plan, hipStream_t stream);
// x bf16 [t, hidden] -> h binary16 [t, inter] -> part float32 [parts][t][hidden] -> y float32 [t, hidden] and, when
// xn is set, xn bf16 [t, hidden] = RMSNorm(y) (cpu-q8 order, identity weight). stream_w: w_gu and w_d in the stream
// layout (launch_stream_layout; the same bits).
void launch_small_layer(const SmallStackPlan& plan, std::size_t t, std::size_t hidden, std::size_t inter, const void* x,
                        const std::int8_t* w_gu, const float* s_gu, const std::int8_t* w_d, const float* s_d, void* h,
                        float* part, float* y, void* xn, double eps, hipStream_t stream, bool stream_w = false);
// The stream layout of an int8 [n, k] weight matrix for the M <= 16 passes (n a multiple of 16, k of 128; n * k
// bytes): each (16-row tile, 128-value group) pair's 2 KB contiguous, in the MFMA operand order of the pass kernels.
// interleave: the gate/up matrix (tiles of 8 gate and 8 up rows, the 64-row interleave).
void launch_stream_layout(const std::int8_t* w, std::size_t ld_w, std::size_t n, std::size_t k, bool interleave, std::int8_t* out,
                          hipStream_t stream);
// The gpu-q8w form: int8 x [t, hidden] with its scales (one per token, or per 128 columns) -> H [t, inter] in h, float32
// per 128 columns, binary16 per token as the large-M per-token stack keeps it (per token also hmax [t, ceil(inter / 8 /
// tiles_per_block)], the partial row maxima of |H|) -> part -> y; when xq_next is
// set, the next layer's input bf16(RMSNorm(y)) goes to xn (bf16) and, quantized, to xq_next / xs_next. stream_w: the
// weights in the stream layout, as for launch_small_layer.
void launch_small_layer_q8(const SmallStackPlan& plan, std::size_t t, std::size_t hidden, std::size_t inter,
                           const std::int8_t* xq, const float* xs, bool per_token, const std::int8_t* w_gu, const float* s_gu,
                           const std::int8_t* w_d, const float* s_d, float* h, float* hmax, float* part, float* y,
                           std::int8_t* xq_next, float* xs_next, void* xn, double eps, hipStream_t stream,
                           bool stream_w = false);

} // namespace sepal::hip
