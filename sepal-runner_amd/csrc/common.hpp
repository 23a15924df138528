// Shared definitions of the HIP kernels of the W8g128 MLP path (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <stdexcept>
#include <mutex>
#include <string>
#include <utility>

#include "sepal_mlp_hip.h"

namespace sepal::hip {

// ---- errors: the C ABI turns these into status codes (the reference's exception types, runner/cuda/src/device.hpp) --

struct InvalidArgument : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};
struct LaunchError : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct IoError : std::runtime_error {      // a packed-weight file cannot be opened, read or written, or is corrupt
    using std::runtime_error::runtime_error;
};
struct StaleError : std::runtime_error {   // a packed-weight file holds other weights (shape, rule, layout, source)
    using std::runtime_error::runtime_error;
};

inline void check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw LaunchError(std::string(what) + ": " + hipGetErrorString(e));
}

inline void require(bool ok, const std::string& message) {
    if (!ok) throw InvalidArgument(message);
}

// Allows `kernel` up to `lds` bytes of dynamic LDS on the current device. The largest size allowed so far is kept per
// (kernel, device) pair, and a mutex orders the check and the attribute call, so launches from several threads or on
// several devices each see the attribute set before their launch.
inline void raise_dynamic_lds(const void* kernel, std::size_t lds, const char* what) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) throw LaunchError(std::string(what) + ": hipGetDevice failed");
    static std::mutex mutex;
    static std::map<std::pair<const void*, int>, std::size_t> raised;
    std::lock_guard<std::mutex> lock(mutex);
    std::size_t& done = raised[{kernel, device}];
    if (lds <= done) return;
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess)
        throw LaunchError(std::string(what) + ": hipFuncSetAttribute(MaxDynamicSharedMemorySize) failed");
    done = lds;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 7u) == 0; }

// ---- vector types of the MFMA builtins ------------------------------------------------------------------------------

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(16 * sizeof(int)))) int i32x16;
typedef __attribute__((__vector_size__(4 * sizeof(unsigned)))) unsigned u32x4;

// ---- element conversions --------------------------------------------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(unsigned short b) { return __uint_as_float(static_cast<unsigned>(b) << 16); }

__device__ __forceinline__ float f16_bits_to_f32(unsigned short b) {
    return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

// float32 -> bfloat16 bits, round to nearest even, NaN kept a quiet NaN (runner/src/cpu/gemm.cpp:73-78).
__device__ __forceinline__ unsigned short f32_to_bf16_bits(float f) {
    const unsigned bits = __float_as_uint(f);
    if ((bits & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<unsigned short>((bits >> 16) | 0x40u);
    return static_cast<unsigned short>((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

// float32 -> binary16 bits, round to nearest even (the hardware conversion) of the float32 value. The empty asm keeps
// the value a rounded float32: otherwise the compiler may fold a producing multiply into a mixed-precision instruction
// that rounds the exact product straight to binary16 (a different result at float32 ties, seen in gemm_s8's output).
__device__ __forceinline__ unsigned short f32_to_f16_bits(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(unsigned short, static_cast<_Float16>(f));
}

// Signed byte `i` of v as a float32, exactly.
__device__ __forceinline__ float s8_at(unsigned v, int i) {
    return static_cast<float>(static_cast<int>(v << (24 - 8 * i)) >> 24);
}

// Four signed bytes -> four bfloat16 in two dwords (low pair, high pair): exact, int8 values have at most 8 significant
// bits. The float is exact and its top 16 bits are the bfloat16.
__device__ __forceinline__ void s8x4_to_bf16x4(unsigned v, unsigned& lo, unsigned& hi) {
    const unsigned f0 = __float_as_uint(s8_at(v, 0)), f1 = __float_as_uint(s8_at(v, 1));
    const unsigned f2 = __float_as_uint(s8_at(v, 2)), f3 = __float_as_uint(s8_at(v, 3));
    lo = __builtin_amdgcn_perm(f1, f0, 0x07060302u);
    hi = __builtin_amdgcn_perm(f3, f2, 0x07060302u);
}

// Four signed bytes -> four binary16 in two dwords, exactly: the byte b + 128 is put under the exponent of 1024 (the
// half 0x6400 | u is 1024 + u) and 1152 = 1024 + 128 is subtracted in binary16, which is exact for these integers.
__device__ __forceinline__ void s8x4_to_f16x4(unsigned v, unsigned& lo, unsigned& hi) {
    const unsigned u = v ^ 0x80808080u;
    const unsigned a = __builtin_amdgcn_perm(0x64646464u, u, 0x07010700u) ;
    const unsigned b = __builtin_amdgcn_perm(0x64646464u, u, 0x07030702u);
    typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 h2;
    const h2 bias = {static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
    const h2 ha = __builtin_bit_cast(h2, a) - bias, hb = __builtin_bit_cast(h2, b) - bias;
    lo = __builtin_bit_cast(unsigned, ha);
    hi = __builtin_bit_cast(unsigned, hb);
}

// ---- silu -----------------------------------------------------------------------------------------------------------

// silu(g) * u as the reference's GPU w8g epilogue writes it: fl(fl(g * exp(-softplus(-g))) * u), softplus(x) =
// max(x, 0) + log1p(exp(-|x|)) (runner/cuda/src/gemm_simt_kernels.cu:27-29), with the HIP device library's expf/log1pf.
__device__ __forceinline__ float swiglu_libm(float g, float u) {
    const float ng = -g;
    const float softplus = fmaxf(ng, 0.0f) + log1pf(expf(-fabsf(ng)));
    return __fmul_rn(__fmul_rn(g, expf(-softplus)), u);
}

// silu(g) * u for the tolerance-pinned w8g epilogue: g * u / (1 + 2^(-g log2 e)) with the hardware exp2 and reciprocal
// (about one ulp each; the result is within a few ulp of silu(g) * u). Large negative g gives 2^(+inf) = inf and a
// reciprocal of 0, so the product is 0; large positive g gives g * u.
__device__ __forceinline__ float swiglu_fast(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
    return (g * u) * __builtin_amdgcn_rcpf(1.0f + e);
}

// exp(x) by Cody-Waite reduction with the two-part ln 2 and the degree-5 polynomial of the cpu-q8 path, with its clamps
// (runner/src/cpu/vmath.hpp:16-32, the Cephes expf method), one lane at a time: every step is one IEEE operation
// or one fused multiply-add, so the result equals the CPU's bit for bit.
__device__ __forceinline__ float exp_cephes(float x) {
    x = x < 88.3762626647949f ? x : 88.3762626647949f;
    x = x > -87.3f ? x : -87.3f;
    const float fx = __builtin_rintf(__fmul_rn(x, 1.44269504088896341f));
    float r = __builtin_fmaf(-fx, 0.693359375f, x);
    r = __builtin_fmaf(-fx, -2.12194440e-4f, r);
    float p = 1.9875691500E-4f;
    p = __builtin_fmaf(p, r, 1.3981999507E-3f);
    p = __builtin_fmaf(p, r, 8.3334519073E-3f);
    p = __builtin_fmaf(p, r, 4.1665795894E-2f);
    p = __builtin_fmaf(p, r, 1.6666665459E-1f);
    p = __builtin_fmaf(p, r, 5.0000001201E-1f);
    p = __builtin_fmaf(p, __fmul_rn(r, r), __fadd_rn(r, 1.0f));
    const unsigned e = static_cast<unsigned>(static_cast<int>(fx) + 127) << 23;
    return __fmul_rn(p, __uint_as_float(e));
}

// silu(g) * u of the cpu-q8 epilogue: (g / (1 + exp(-g))) * u (runner/src/cpu/vmath.hpp:35-38, gemm.cpp:427-430).
__device__ __forceinline__ float swiglu_cephes(float g, float u) {
    const float e = exp_cephes(__fsub_rn(0.0f, g));
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), u);
}

// silu(g) * u of the gpu-q8w multiplies. With one activation scale per 128 values (cpu-q8's I8_Z blocking) the
// cpu-q8 epilogue bit for bit; with one scale per token, a form with no reference bits to match, the fast one (the
// float results are held to the parity bar; the int32 group sums stay exact).
template <bool PER_TOKEN>
__device__ __forceinline__ float swiglu_q8(float g, float u) {
    if constexpr (PER_TOKEN) return swiglu_fast(g, u);
    else return swiglu_cephes(g, u);
}

// ---- group scales in Horner form ---------------------------------------------------------------------------------------

// One Horner step of the w8g group scales. The MFMAs add each group's partial sum P_g straight into the running sum U,
// which is kept in units of the current group's effective scale e: U_g = U_{g-1} * (e_{g-1} / e_g) + P_g, and the output
// is U_last * e_last (the identity Y = sum_g s_g P_g). Returns the factor e_{g-1} / e_g and advances e to the group of
// scale s:
//   - s <= 0 (or NaN) marks an all-zero group (P_g = 0): e is kept and the factor is 1;
//   - otherwise e_g = max(s, 2^-60 * emax, 2^-126), emax the largest scale so far (0 before the first). The floor keeps
//     the factor at most 2^60 and e_g normal, so U stays finite for any finite X (|U| <= 2^60 * 127 * K * max|x|) and
//     the reciprocal never overflows. A group raised by the floor counts as if its scale were e_g: the difference,
//     |P_g| * (e_g - s) <= 127 * 128 * max|x| * 2^-60 * emax, is below the rounding of the groups near emax (and, at the
//     2^-126 floor, below the smallest normal float32 times 2^14 max|x|).
__device__ __forceinline__ float horner_step(float s, float& e, float& emax) {
    const float lo = fmaxf(emax * 0x1p-60f, 0x1p-126f);
    const float en = s > 0.0f ? fmaxf(s, lo) : e;
    emax = fmaxf(emax, s > 0.0f ? en : 0.0f);
    const float ratio = __fmul_rn(e, __builtin_amdgcn_rcpf(en));
    e = en;
    return ratio;
}

// ---- output stores by type ------------------------------------------------------------------------------------------

template <int YT>
__device__ __forceinline__ void store_out(void* y, std::size_t idx, float v) {
    if constexpr (YT == SEPAL_HIP_F32) {
        static_cast<float*>(y)[idx] = v;
    } else if constexpr (YT == SEPAL_HIP_BF16) {
        static_cast<unsigned short*>(y)[idx] = f32_to_bf16_bits(v);
    } else {
        static_cast<unsigned short*>(y)[idx] = f32_to_f16_bits(v);
    }
}

inline std::size_t elem_bytes(int type) { return type == SEPAL_HIP_F32 ? 4 : 2; }

// ---- workspaces (library-owned scratch: split-K partials and counters, converted operands) ---------------------------

// Layout of a workspace: [0, kCounterBytes) split-K arrival counters (zero at rest: the last block of a column block
// resets its counter), then kPartialBytes of split-K partial sums, then the scratch of the entry point.
inline constexpr std::size_t kCounterBytes = std::size_t{64} << 10;
inline constexpr std::size_t kPartialBytes = std::size_t{32} << 20;
inline constexpr std::size_t kScratchOffset = kCounterBytes + kPartialBytes;

// The workspace of (current device, stream), at least `bytes` long (zero-filled when first allocated or grown; a grown
// one waits for `stream` before the old one is freed), held for the lifetime of the lease: an entry point takes one
// lease for all the work it enqueues.
class Lease {
public:
    Lease(std::size_t bytes, hipStream_t stream);
    char* base() const { return base_; }

private:
    std::unique_lock<std::mutex> lock_;
    char* base_ = nullptr;
};

} // namespace sepal::hip
