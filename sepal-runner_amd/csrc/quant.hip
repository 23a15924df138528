// Quantizers and glue kernels of the W8g128 MLP path (HBM-bound, one pass each).
//
//   quantize_group: the load-time weight packer and the per-128 activation quantizer. 16 lanes own one (row, 128-group)
//     (8 values each, one 16- or 32-byte load), the group maximum is a 16-lane butterfly (exact in any order), each
//     value is quantized on its own, 8 bytes are stored per lane. Rule DIVIDE restates quantize_group_s8_kernel
//     (runner/cuda/src/gemm_simt_kernels.cu:266-286), rule RECIPROCAL the cpu-q8 quantise (runner/src/cpu/gemm.cpp:
//     103-106, 141-163, 288-303). With a second source the rows are read in the 64-row gate/up interleave
//     (gemm_simt_kernels.hpp:72-77).
//   quantize_rows_token: one scale per row (block = cols), rule RECIPROCAL; a block of 256 threads per row.
//   rmsnorm: the cpu-q8 RMSNorm with its exact summation order (runner/src/cpu/elementwise.cpp:22-59): 32 lanes stand
//     for the reference's 4 x 8 accumulator lanes, then the same combining order. Its fused variant rounds the output to
//     bfloat16 and quantizes it in the same pass (the layer input of the q8 stack: RMSNorm, bf16, quantize_rows).
#include "common.hpp"
#include "gemm_kernels.hpp"

namespace sepal::hip {
namespace quant {

template <int ST>
__device__ __forceinline__ void load8(const void* base, std::size_t idx, float (&v)[8]) {
    if constexpr (ST == SEPAL_HIP_F32) {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
        const float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const u32x4 u = *reinterpret_cast<const u32x4*>(static_cast<const unsigned short*>(base) + idx);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const unsigned short lo = static_cast<unsigned short>(u[i] & 0xFFFFu), hi = static_cast<unsigned short>(u[i] >> 16);
            if constexpr (ST == SEPAL_HIP_BF16) {
                v[2 * i] = bf16_bits_to_f32(lo);
                v[2 * i + 1] = bf16_bits_to_f32(hi);
            } else {
                v[2 * i] = f16_bits_to_f32(lo);
                v[2 * i + 1] = f16_bits_to_f32(hi);
            }
        }
    }
}

template <int RULE>
__device__ __forceinline__ int quantize_value(float w, float scale, float inverse) {
    if constexpr (RULE == SEPAL_HIP_RULE_DIVIDE) {
        if (!(scale > 0.0f)) return 0;
        // rint(w / scale) with the IEEE quotient. With inverse = rcp(scale) (within 1 ulp; 0 when not usable) and
        // |w / scale| <= 127, t = w * inverse is within 2^-15 of the quotient; when t is more than 2^-12 from a
        // half-integer, the quotient lies in the same rounding interval, so rint(t) is its rint. Otherwise (or for a
        // NaN) the division decides.
        const float t = __fmul_rn(w, inverse), rt = __builtin_rintf(t);
        const float r = inverse != 0.0f && fabsf(fabsf(__fsub_rn(t, rt)) - 0.5f) > 0x1p-12f ? rt
                                                                                         : __builtin_rintf(__fdiv_rn(w, scale));
        return static_cast<int>(fminf(fmaxf(r, -127.0f), 127.0f));
    } else {
        float r = __builtin_rintf(__fmul_rn(w, inverse));
        r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
        return static_cast<int>(r);
    }
}

template <int ST, int RULE, int LANES>
__global__ void __launch_bounds__(256) quantize_group_kernel(const void* __restrict__ src, std::size_t ld_src,
                                                             const void* __restrict__ src_up, std::int8_t* __restrict__ q,
                                                             std::size_t ld_q, float* __restrict__ s, std::size_t ld_s,
                                                             std::size_t rows, std::size_t groups, std::size_t inter) {
    // LANES lanes per (row, group); lane `sub` holds the 8-value chunks sub, sub + LANES, ...
    constexpr int CH = 16 / LANES;
    const std::size_t gid = (static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x) / LANES;
    const int sub = threadIdx.x % LANES;
    const bool live = gid < rows * groups;
    const std::size_t row = live ? gid / groups : 0, g = live ? gid % groups : 0;
    // source row: plain, or the 64-row gate/up interleave of the fused SwiGLU weights
    const void* base = src;
    std::size_t srow = row;
    if (src_up != nullptr) {
        const std::size_t b = row / 128, r = row % 128;
        if (r < 64) srow = 64 * b + r;
        else {
            srow = 64 * b + (r - 64);
            base = src_up;
        }
    }
    float v[CH][8];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        if (live) load8<ST>(base, srow * ld_src + g * 128 + (sub + LANES * c) * 8, v[c]);
        else
#pragma unroll
            for (int i = 0; i < 8; ++i) v[c][i] = 0.0f;
    }
    float m = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float a = fabsf(v[c][i]);
            m = a > m ? a : m;
        }
#pragma unroll
    for (int o = LANES / 2; o > 0; o >>= 1) {
        const float other = __shfl_xor(m, o, LANES);
        m = other > m ? other : m;
    }
    float scale, inverse = 0.0f;
    if constexpr (RULE == SEPAL_HIP_RULE_DIVIDE) {
        scale = __fdiv_rn(m, 127.0f);
        // (the fast path of quantize_value: scales whose reciprocal is a normal float; inf and NaN take the division)
        if (scale >= 0x1p-100f && scale <= 0x1p100f) inverse = __builtin_amdgcn_rcpf(scale);
    } else {
        scale = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
        inverse = __fdiv_rn(1.0f, scale);
    }
    if (!live) return;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        unsigned packed[2] = {0u, 0u};
#pragma unroll
        for (int i = 0; i < 8; ++i)
            packed[i / 4] |= (static_cast<unsigned>(quantize_value<RULE>(v[c][i], scale, inverse)) & 0xFFu) << (8 * (i % 4));
        *reinterpret_cast<uint2*>(q + row * ld_q + g * 128 + (sub + LANES * c) * 8) = make_uint2(packed[0], packed[1]);
    }
    if (sub == 0) s[row * ld_s + g] = scale;
}

// One scale per row: the row maximum (block reduction), then the quantization (rule RECIPROCAL). Rows of up to
// 256 * kTokChunks chunks of 8 values stay in registers between the two (every load in flight at once); longer rows
// are read twice.
constexpr int kTokChunks = 8;

template <int ST>
__global__ void __launch_bounds__(256) quantize_rows_token_kernel(const void* __restrict__ x, std::size_t ld_x,
                                                                  std::int8_t* __restrict__ q, std::size_t ld_q,
                                                                  float* __restrict__ scales, std::size_t ld_s, int cols) {
    __shared__ float red[4];
    const std::size_t row = blockIdx.x;
    const int chunks = cols / 8;
    const auto block_max = [&](float m) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float other = __shfl_xor(m, o, 64);
            m = other > m ? other : m;
        }
        if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = m;
        __syncthreads();
        m = red[0];
#pragma unroll
        for (int i = 1; i < 4; ++i) m = red[i] > m ? red[i] : m;
        return m;
    };
    if (ST != SEPAL_HIP_F32 && chunks <= 256 * kTokChunks) {
        // 16-bit rows stay in registers as loaded (half the registers of the float32 values) and are widened twice,
        // for the maximum and for the quantization: 84-85 against 89-92 us at C4's H (15872 x 9728), same bits
        u32x4 raw[kTokChunks];
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < kTokChunks; ++j) {
            const int c = threadIdx.x + 256 * j;
            raw[j] = c < chunks ? *reinterpret_cast<const u32x4*>(static_cast<const unsigned short*>(x) + row * ld_x + 8 * c) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int j = 0; j < kTokChunks; ++j) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const unsigned short b = static_cast<unsigned short>(raw[j][i / 2] >> (16 * (i % 2)));
                const float a = fabsf(ST == SEPAL_HIP_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b));
                m = a > m ? a : m;
            }
        }
        m = block_max(m);
        const float scale = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
        const float inverse = __fdiv_rn(1.0f, scale);
        if (threadIdx.x == 0) scales[row * ld_s] = scale;
#pragma unroll
        for (int j = 0; j < kTokChunks; ++j) {
            const int c = threadIdx.x + 256 * j;
            if (c >= chunks) continue;
            unsigned packed[2] = {0u, 0u};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const unsigned short b = static_cast<unsigned short>(raw[j][i / 2] >> (16 * (i % 2)));
                const float v = ST == SEPAL_HIP_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
                packed[i / 4] |= (static_cast<unsigned>(quantize_value<SEPAL_HIP_RULE_RECIPROCAL>(v, scale, inverse)) & 0xFFu) << (8 * (i % 4));
            }
            *reinterpret_cast<uint2*>(q + row * ld_q + 8 * c) = make_uint2(packed[0], packed[1]);
        }
        return;
    }
    if (chunks <= 256 * kTokChunks) {
        float v[kTokChunks][8];
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < kTokChunks; ++j) {
            const int c = threadIdx.x + 256 * j;
            if (c < chunks) {
                load8<ST>(x, row * ld_x + 8 * c, v[j]);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[j][i] = 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float a = fabsf(v[j][i]);
                m = a > m ? a : m;
            }
        }
        m = block_max(m);
        const float scale = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
        const float inverse = __fdiv_rn(1.0f, scale);
        if (threadIdx.x == 0) scales[row * ld_s] = scale;
#pragma unroll
        for (int j = 0; j < kTokChunks; ++j) {
            const int c = threadIdx.x + 256 * j;
            if (c >= chunks) continue;
            unsigned packed[2] = {0u, 0u};
#pragma unroll
            for (int i = 0; i < 8; ++i)
                packed[i / 4] |= (static_cast<unsigned>(quantize_value<SEPAL_HIP_RULE_RECIPROCAL>(v[j][i], scale, inverse)) & 0xFFu) << (8 * (i % 4));
            *reinterpret_cast<uint2*>(q + row * ld_q + 8 * c) = make_uint2(packed[0], packed[1]);
        }
        return;
    }
    float m = 0.0f;
    for (int c = threadIdx.x; c < chunks; c += 256) {
        float v[8];
        load8<ST>(x, row * ld_x + 8 * c, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float a = fabsf(v[i]);
            m = a > m ? a : m;
        }
    }
    m = block_max(m);
    const float scale = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
    const float inverse = __fdiv_rn(1.0f, scale);
    if (threadIdx.x == 0) scales[row * ld_s] = scale;
    for (int c = threadIdx.x; c < chunks; c += 256) {
        float v[8];
        load8<ST>(x, row * ld_x + 8 * c, v);
        unsigned packed[2] = {0u, 0u};
#pragma unroll
        for (int i = 0; i < 8; ++i)
            packed[i / 4] |= (static_cast<unsigned>(quantize_value<SEPAL_HIP_RULE_RECIPROCAL>(v[i], scale, inverse)) & 0xFFu) << (8 * (i % 4));
        *reinterpret_cast<uint2*>(q + row * ld_q + 8 * c) = make_uint2(packed[0], packed[1]);
    }
}

// The same rule for rows of any length and stride (kernel_i8_y's packing takes any K, runner/src/cpu/gemm.cpp:
// 286-306): element loads, the row maximum by the same block reduction (a maximum does not depend on order), then each
// value quantized on its own, so the bits are those of the vector kernel.
template <int ST>
__global__ void __launch_bounds__(256) quantize_rows_token_any_kernel(const void* __restrict__ x, std::size_t ld_x,
                                                                      std::int8_t* __restrict__ q, std::size_t ld_q,
                                                                      float* __restrict__ scales, std::size_t ld_s, int cols) {
    __shared__ float red[4];
    const std::size_t row = blockIdx.x;
    const auto at = [&](int c) -> float {
        const std::size_t i = row * ld_x + c;
        if constexpr (ST == SEPAL_HIP_F32) return static_cast<const float*>(x)[i];
        else if constexpr (ST == SEPAL_HIP_BF16) return bf16_bits_to_f32(static_cast<const unsigned short*>(x)[i]);
        else return f16_bits_to_f32(static_cast<const unsigned short*>(x)[i]);
    };
    float m = 0.0f;
    for (int c = threadIdx.x; c < cols; c += 256) {
        const float a = fabsf(at(c));
        m = a > m ? a : m;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float other = __shfl_xor(m, o, 64);
        m = other > m ? other : m;
    }
    if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) m = red[i] > m ? red[i] : m;
    const float scale = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
    const float inverse = __fdiv_rn(1.0f, scale);
    if (threadIdx.x == 0) scales[row * ld_s] = scale;
    for (int c = threadIdx.x; c < cols; c += 256)
        q[row * ld_q + c] = static_cast<std::int8_t>(quantize_value<SEPAL_HIP_RULE_RECIPROCAL>(at(c), scale, inverse));
}

// One row per wave, four rows per block. The row is read coalesced (16 bytes per lane, every load of a segment in flight
// at once) into LDS, then lanes 0..31 run the reference's 32 accumulator chains from LDS: lane L is accumulator register
// L / 8, lane L % 8, and adds x[c]^2 for c = L, L + 32, ... in order (then, for a tail of 8 to 31 columns, lanes 0..7
// take the remaining groups of 8). The combine and the normalising pass follow the reference.
constexpr int kNormSeg = 2560;  // columns per LDS segment and wave (a whole row of the MLP width)
static_assert(kNormSeg % 512 == 0, "a segment is loaded in rounds of 512 columns (8 per lane)");

// OUT: NORM_STORE writes y (YT); NORM_Q_TOKEN and NORM_Q_128 round each value to bfloat16 (y, when not null, gets those
// bits) and quantize the rounded values as quantize_rows does (one scale per row, or per 128 columns).
enum { NORM_STORE = 0, NORM_Q_TOKEN = 1, NORM_Q_128 = 2 };

template <int YT, int OUT>
__global__ void __launch_bounds__(256) rmsnorm_kernel(const float* __restrict__ x, std::size_t ld_x, void* __restrict__ y,
                                                      std::size_t ld_y, const float* __restrict__ w1, int rows, int cols,
                                                      double eps, std::int8_t* __restrict__ q, std::size_t ld_q,
                                                      float* __restrict__ qs, std::size_t ld_qs) {
    __shared__ __align__(16) float seg[4][kNormSeg];
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, L = lane % 32;
    const int row = blockIdx.x * 4 + wave;
    const bool live = row < rows;
    const float* xr = x + static_cast<std::size_t>(live ? row : 0) * ld_x;
    float* buf = seg[wave];
    float a = 0.0f;
    const int full = cols / 32 * 32;  // columns taken by the 32-wide loop
    // len is a multiple of 8: 8-column pieces, one per lane and round, loads first. When the row is one segment, v
    // still holds it for the normalising pass.
    constexpr int R = kNormSeg / 8 / 64;
    float4 v[R][2];
    for (int s0 = 0; s0 < cols; s0 += kNormSeg) {
        const int len = min(kNormSeg, cols - s0);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int c = 8 * (lane + 64 * r);
            const int cc = min(c, len - 8);  // clamped: in bounds, never stored
            v[r][0] = *reinterpret_cast<const float4*>(xr + s0 + cc);
            v[r][1] = *reinterpret_cast<const float4*>(xr + s0 + cc + 4);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int c = 8 * (lane + 64 * r);
            if (c < len) {
                *reinterpret_cast<float4*>(buf + c) = v[r][0];
                *reinterpret_cast<float4*>(buf + c + 4) = v[r][1];
            }
        }
        __syncthreads();
        if (lane < 32) {
            const int end32 = min(len, full - s0);  // this segment's part of the 32-wide loop
            int c = 0;
            // eight reads in flight, then their eight links of the chain, in order
            for (; c + 256 <= end32; c += 256) {
                float v8[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v8[u] = buf[c + 32 * u + L];
#pragma unroll
                for (int u = 0; u < 8; ++u) a = __builtin_fmaf(v8[u], v8[u], a);
            }
            for (; c + 32 <= end32; c += 32) {
                const float e = buf[c + L];
                a = __builtin_fmaf(e, e, a);
            }
            if (s0 + len == cols) {  // the tail after the 32-wide loop, in groups of 8 on lanes 0..7
                for (c = end32 > 0 ? end32 : full - s0; c + 8 <= len; c += 8)
                    if (L < 8) {
                        const float e = buf[c + L];
                        a = __builtin_fmaf(e, e, a);
                    }
            }
        }
        __syncthreads();
    }
    const int l8 = L % 8;
    const float a0 = __shfl(a, l8), a1 = __shfl(a, 8 + l8), a2 = __shfl(a, 16 + l8), a3 = __shfl(a, 24 + l8);
    const float sl = __fadd_rn(__fadd_rn(a0, a1), __fadd_rn(a2, a3));  // s[l8] on every lane
    const float sl4 = __shfl(sl, (l8 + 4) % 8);
    const float h = __fadd_rn(sl, sl4);                                 // h[l8 % 4] on lanes l8 < 4
    const float h0 = __shfl(h, 0), h1 = __shfl(h, 1), h2 = __shfl(h, 2), h3 = __shfl(h, 3);
    const float sum = __fadd_rn(__fadd_rn(h0, h2), __fadd_rn(h1, h3));
    if (!live) return;
    const double mean = static_cast<double>(sum) / static_cast<double>(cols);
    const float inv = static_cast<float>(1.0 / __builtin_sqrt(mean + eps));
    if constexpr (OUT == NORM_STORE) {
        const bool vec_out = reinterpret_cast<std::uintptr_t>(y) % 16 == 0 && ld_y * (YT == SEPAL_HIP_F32 ? 4 : 2) % 16 == 0 &&
                             (w1 == nullptr || reinterpret_cast<std::uintptr_t>(w1) % 16 == 0);
        if (cols <= kNormSeg && vec_out) {
            // from the registers: lane l holds columns 8 (l + 64 r) .. + 7; one 16-byte (or two, float32) store each
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int c = 8 * (lane + 64 * r);
                if (c >= cols) continue;
                const float vv[8] = {v[r][0].x, v[r][0].y, v[r][0].z, v[r][0].w, v[r][1].x, v[r][1].y, v[r][1].z, v[r][1].w};
                float g[8] = {1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f};
                if (w1 != nullptr) {
                    const float4 g0 = *reinterpret_cast<const float4*>(w1 + c), g1 = *reinterpret_cast<const float4*>(w1 + c + 4);
                    g[0] = g0.x; g[1] = g0.y; g[2] = g0.z; g[3] = g0.w;
                    g[4] = g1.x; g[5] = g1.y; g[6] = g1.z; g[7] = g1.w;
                }
                float n[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) n[j] = __fmul_rn(__fmul_rn(vv[j], inv), g[j]);
                if constexpr (YT == SEPAL_HIP_F32) {
                    float* yr = static_cast<float*>(y) + static_cast<std::size_t>(row) * ld_y + c;
                    *reinterpret_cast<float4*>(yr) = make_float4(n[0], n[1], n[2], n[3]);
                    *reinterpret_cast<float4*>(yr + 4) = make_float4(n[4], n[5], n[6], n[7]);
                } else {
                    unsigned u[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const unsigned lo = YT == SEPAL_HIP_BF16 ? f32_to_bf16_bits(n[2 * j]) : f32_to_f16_bits(n[2 * j]);
                        const unsigned hi = YT == SEPAL_HIP_BF16 ? f32_to_bf16_bits(n[2 * j + 1]) : f32_to_f16_bits(n[2 * j + 1]);
                        u[j] = lo | (hi << 16);
                    }
                    *reinterpret_cast<u32x4*>(static_cast<unsigned short*>(y) + static_cast<std::size_t>(row) * ld_y + c) =
                        u32x4{u[0], u[1], u[2], u[3]};
                }
            }
            return;
        }
        for (int c = 4 * lane; c < cols; c += 256) {
            const float4 v = *reinterpret_cast<const float4*>(xr + c);
            const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (c + j < cols)
                    store_out<YT>(y, static_cast<std::size_t>(row) * ld_y + c + j,
                                  __fmul_rn(__fmul_rn(vv[j], inv), w1 != nullptr ? w1[c + j] : 1.0f));
        }
    } else {
        // four normalised columns c .. c + 3 rounded to bfloat16 (zero past cols)
        const auto norm4 = [&](int c, float (&b)[4]) {
            if (c < cols) {
                const float4 v = *reinterpret_cast<const float4*>(xr + c);
                const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float n = __fmul_rn(__fmul_rn(vv[j], inv), w1 != nullptr ? w1[c + j] : 1.0f);
                    b[j] = bf16_bits_to_f32(f32_to_bf16_bits(n));
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) b[j] = 0.0f;
            }
        };
        const auto amax4 = [](const float (&b)[4], float m) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float a = fabsf(b[j]);
                m = a > m ? a : m;
            }
            return m;
        };
        const auto put4 = [&](int c, const float (&b)[4], float scale, float inverse) {
            unsigned packed = 0u;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                packed |= (static_cast<unsigned>(quantize_value<SEPAL_HIP_RULE_RECIPROCAL>(b[j], scale, inverse)) & 0xFFu) << (8 * j);
            *reinterpret_cast<unsigned*>(q + static_cast<std::size_t>(row) * ld_q + c) = packed;
            if (y != nullptr) {
                unsigned short* yb = static_cast<unsigned short*>(y) + static_cast<std::size_t>(row) * ld_y + c;
#pragma unroll
                for (int j = 0; j < 4; ++j) yb[j] = f32_to_bf16_bits(b[j]);
            }
        };
        const bool vec_q = reinterpret_cast<std::uintptr_t>(q) % 8 == 0 && ld_q % 8 == 0 &&
                           (y == nullptr || (reinterpret_cast<std::uintptr_t>(y) % 16 == 0 && ld_y % 8 == 0)) &&
                           (w1 == nullptr || reinterpret_cast<std::uintptr_t>(w1) % 16 == 0);
        if (cols <= kNormSeg && vec_q) {
            // from the registers: lane l holds columns 8 (l + 64 r) .. + 7, a 128-column block is 16 lanes of one r
            float nb[R][8];
            float m = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int c = 8 * (lane + 64 * r);
                const float vv[8] = {v[r][0].x, v[r][0].y, v[r][0].z, v[r][0].w, v[r][1].x, v[r][1].y, v[r][1].z, v[r][1].w};
                float g[8] = {1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f};
                if (w1 != nullptr && c < cols) {
                    const float4 g0 = *reinterpret_cast<const float4*>(w1 + c), g1 = *reinterpret_cast<const float4*>(w1 + c + 4);
                    g[0] = g0.x; g[1] = g0.y; g[2] = g0.z; g[3] = g0.w;
                    g[4] = g1.x; g[5] = g1.y; g[6] = g1.z; g[7] = g1.w;
                }
                float mr = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    nb[r][j] = c < cols ? bf16_bits_to_f32(f32_to_bf16_bits(__fmul_rn(__fmul_rn(vv[j], inv), g[j]))) : 0.0f;
                    const float a = fabsf(nb[r][j]);
                    mr = a > mr ? a : mr;
                }
                if constexpr (OUT == NORM_Q_128) {
#pragma unroll
                    for (int o = 8; o > 0; o >>= 1) {
                        const float other = __shfl_xor(mr, o, 16);
                        mr = other > mr ? other : mr;
                    }
                    const float scale = mr > 0.0f ? __fdiv_rn(mr, 127.0f) : 1.0f;
                    const float inverse = __fdiv_rn(1.0f, scale);
                    if (c < cols) {
                        unsigned packed[2] = {0u, 0u};
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            packed[j / 4] |= (static_cast<unsigned>(quantize_value<SEPAL_HIP_RULE_RECIPROCAL>(nb[r][j], scale, inverse)) & 0xFFu)
                                             << (8 * (j % 4));
                        *reinterpret_cast<uint2*>(q + static_cast<std::size_t>(row) * ld_q + c) = make_uint2(packed[0], packed[1]);
                        if (lane % 16 == 0) qs[static_cast<std::size_t>(row) * ld_qs + c / 128] = scale;
                    }
                } else {
                    m = mr > m ? mr : m;
                }
            }
            float scale = 1.0f, inverse = 1.0f;
            if constexpr (OUT == NORM_Q_TOKEN) {
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) {
                    const float other = __shfl_xor(m, o, 64);
                    m = other > m ? other : m;
                }
                scale = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
                inverse = __fdiv_rn(1.0f, scale);
                if (lane == 0) qs[static_cast<std::size_t>(row) * ld_qs] = scale;
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int c = 8 * (lane + 64 * r);
                if (c >= cols) continue;
                if constexpr (OUT == NORM_Q_TOKEN) {
                    unsigned packed[2] = {0u, 0u};
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        packed[j / 4] |= (static_cast<unsigned>(quantize_value<SEPAL_HIP_RULE_RECIPROCAL>(nb[r][j], scale, inverse)) & 0xFFu)
                                         << (8 * (j % 4));
                    *reinterpret_cast<uint2*>(q + static_cast<std::size_t>(row) * ld_q + c) = make_uint2(packed[0], packed[1]);
                }
                if (y != nullptr) {
                    unsigned u[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        u[j] = static_cast<unsigned>(f32_to_bf16_bits(nb[r][2 * j])) | (static_cast<unsigned>(f32_to_bf16_bits(nb[r][2 * j + 1])) << 16);
                    *reinterpret_cast<u32x4*>(static_cast<unsigned short*>(y) + static_cast<std::size_t>(row) * ld_y + c) =
                        u32x4{u[0], u[1], u[2], u[3]};
                }
            }
            return;
        }
        if constexpr (OUT == NORM_Q_128) {
            // lanes 0..31 hold one 128-column block, lanes 32..63 the next (cols is a multiple of 128)
            for (int c0 = 0; c0 < cols; c0 += 256) {
                const int c = c0 + 4 * lane;
                float b[4];
                norm4(c, b);
                float m = amax4(b, 0.0f);
#pragma unroll
                for (int o = 16; o > 0; o >>= 1) {
                    const float other = __shfl_xor(m, o, 32);
                    m = other > m ? other : m;
                }
                const float scale = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
                const float inverse = __fdiv_rn(1.0f, scale);
                if (c < cols) {
                    put4(c, b, scale, inverse);
                    if (lane % 32 == 0) qs[static_cast<std::size_t>(row) * ld_qs + c / 128] = scale;
                }
            }
        } else {
            float m = 0.0f;
            for (int c = 4 * lane; c < cols; c += 256) {
                float b[4];
                norm4(c, b);
                m = amax4(b, m);
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float other = __shfl_xor(m, o, 64);
                m = other > m ? other : m;
            }
            const float scale = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
            const float inverse = __fdiv_rn(1.0f, scale);
            if (lane == 0) qs[static_cast<std::size_t>(row) * ld_qs] = scale;
            for (int c = 4 * lane; c < cols; c += 256) {
                float b[4];
                norm4(c, b);
                put4(c, b, scale, inverse);
            }
        }
    }
}

__global__ void f32_to_bf16_kernel(const float* __restrict__ src, std::uint16_t* __restrict__ dst, std::size_t count) {
    const std::size_t i = static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < count) dst[i] = f32_to_bf16_bits(src[i]);
}

// The GPU int8 path's per-row quantizer (the int8-activation multiply's rows, and per-output-channel weights):
// v = x * smooth[c] in float32 when smooth is set; amax = max |v| over the row; scale = amax / 127 (0 for an all-zero
// row); q = clamp(rint(v * (127 / amax)), -127, 127), 0 when amax is 0. One block per row: the maximum (order-free),
// then the values (runner/cuda/src/gemm_s8_kernels.cu:29-32, 50-79, 82-110; host form
// runner/cuda/tests/test_gemm_s8_kernels.cpp:58-68).
template <int ST>
__global__ void __launch_bounds__(256) s8_rows_kernel(const void* __restrict__ x, std::size_t ld_x, const float* __restrict__ smooth,
                                                      std::int8_t* __restrict__ q, std::size_t ld_q, float* __restrict__ scales,
                                                      int cols) {
    __shared__ float red[4];
    const std::size_t row = blockIdx.x;
    const int chunks = cols / 8;
    const auto values = [&](int c, float (&v)[8]) {
        load8<ST>(x, row * ld_x + 8 * c, v);
        if (smooth != nullptr)
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = __fmul_rn(v[i], smooth[8 * c + i]);
    };
    float m = 0.0f;
    for (int c = threadIdx.x; c < chunks; c += 256) {
        float v[8];
        values(c, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float inv = m > 0.0f ? __fdiv_rn(127.0f, m) : 0.0f;
    if (threadIdx.x == 0) scales[row] = __fdiv_rn(m, 127.0f);
    for (int c = threadIdx.x; c < chunks; c += 256) {
        float v[8];
        values(c, v);
        unsigned packed[2] = {0u, 0u};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float r = __builtin_rintf(__fmul_rn(v[i], inv));
            r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
            packed[i / 4] |= (static_cast<unsigned>(static_cast<int>(r)) & 0xFFu) << (8 * (i % 4));
        }
        *reinterpret_cast<uint2*>(q + row * ld_q + 8 * c) = make_uint2(packed[0], packed[1]);
    }
}

// Calibration statistics of binary16 activations, one thread per column, the rows in order (so every run gives the
// same bits): m = max |x[r, c]|; with STATS also a = sum |x[r, c]| and q = sum x[r, c]^2 in double, added into what
// is there (runner/cuda/src/gemm_s8_kernels.cu:121-149).
template <bool STATS>
__global__ void __launch_bounds__(256) column_stats_kernel(const std::uint16_t* __restrict__ x, std::size_t ld_x, std::size_t rows,
                                                           int cols, float* __restrict__ amax, double* __restrict__ sums) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= cols) return;
    float m = 0.0f;
    double a = 0.0, q = 0.0;
    for (std::size_t r = 0; r < rows; ++r) {
        const float v = f16_bits_to_f32(x[r * ld_x + c]);
        m = fmaxf(m, fabsf(v));
        if constexpr (STATS) {
            a = __dadd_rn(a, static_cast<double>(fabsf(v)));
            q = __dadd_rn(q, __dmul_rn(static_cast<double>(v), static_cast<double>(v)));
        }
    }
    if constexpr (STATS) {
        amax[c] = fmaxf(amax[c], m);
        sums[c] = __dadd_rn(sums[c], a);
        sums[cols + c] = __dadd_rn(sums[cols + c], q);
    } else {
        amax[c] = m;
    }
}

// s[r][g] = sw[r] for g < groups: a per-channel scale as per-group scales
__global__ void broadcast_scales_kernel(const float* __restrict__ sw, float* __restrict__ s, std::size_t n, std::size_t groups) {
    const std::size_t i = static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n * groups) s[i] = sw[i / groups];
}

__global__ void f32_to_f16_kernel(const float* __restrict__ src, std::size_t ld_src, std::uint16_t* __restrict__ dst,
                                  std::size_t ld_dst, std::size_t rows, std::size_t cols) {
    const std::size_t i = static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < rows * cols) dst[(i / cols) * ld_dst + i % cols] = f32_to_f16_bits(src[(i / cols) * ld_src + i % cols]);
}

template <int ST>
void launch_group(const void* src, std::size_t ld_src, const void* src_up, std::int8_t* q, std::size_t ld_q, float* s,
                  std::size_t ld_s, std::size_t rows, std::size_t k, int rule, std::size_t inter, hipStream_t stream) {
    const std::size_t groups = k / 128;
    constexpr int kLanes = 8;
    const std::size_t blocks = (rows * groups * kLanes + 255) / 256;
    if (rule == SEPAL_HIP_RULE_DIVIDE)
        quantize_group_kernel<ST, SEPAL_HIP_RULE_DIVIDE, kLanes><<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(
            src, ld_src, src_up, q, ld_q, s, ld_s, rows, groups, inter);
    else
        quantize_group_kernel<ST, SEPAL_HIP_RULE_RECIPROCAL, kLanes><<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(
            src, ld_src, src_up, q, ld_q, s, ld_s, rows, groups, inter);
    check_launch("quantize_group kernel launch");
}

} // namespace quant

void launch_quantize_group(const void* src, int src_type, std::size_t ld_src, const void* src_up, std::int8_t* q,
                           std::size_t ld_q, float* s, std::size_t ld_s, std::size_t rows, std::size_t k, int rule,
                           std::size_t inter, hipStream_t stream) {
    switch (src_type) {
    case SEPAL_HIP_F32: quant::launch_group<SEPAL_HIP_F32>(src, ld_src, src_up, q, ld_q, s, ld_s, rows, k, rule, inter, stream); break;
    case SEPAL_HIP_BF16: quant::launch_group<SEPAL_HIP_BF16>(src, ld_src, src_up, q, ld_q, s, ld_s, rows, k, rule, inter, stream); break;
    default: quant::launch_group<SEPAL_HIP_F16>(src, ld_src, src_up, q, ld_q, s, ld_s, rows, k, rule, inter, stream); break;
    }
}

void launch_quantize_rows(const void* x, int x_type, std::size_t ld_x, std::int8_t* q, std::size_t ld_q, float* scales,
                          std::size_t ld_s, std::size_t rows, std::size_t cols, std::size_t block, hipStream_t stream) {
    if (block == 128) {
        launch_quantize_group(x, x_type, ld_x, nullptr, q, ld_q, scales, ld_s, rows, cols, SEPAL_HIP_RULE_RECIPROCAL, 0, stream);
        return;
    }
    const dim3 grid(static_cast<unsigned>(rows));
    const std::size_t eb = x_type == SEPAL_HIP_F32 ? 4 : 2;
    if (cols % 16 != 0 || ld_x % 16 != 0 || ld_q % 16 != 0 || reinterpret_cast<std::uintptr_t>(x) % 16 != 0 ||
        reinterpret_cast<std::uintptr_t>(q) % 16 != 0 || (ld_x * eb) % 16 != 0) {
        switch (x_type) {
        case SEPAL_HIP_F32: quant::quantize_rows_token_any_kernel<SEPAL_HIP_F32><<<grid, dim3(256), 0, stream>>>(x, ld_x, q, ld_q, scales, ld_s, static_cast<int>(cols)); break;
        case SEPAL_HIP_BF16: quant::quantize_rows_token_any_kernel<SEPAL_HIP_BF16><<<grid, dim3(256), 0, stream>>>(x, ld_x, q, ld_q, scales, ld_s, static_cast<int>(cols)); break;
        default: quant::quantize_rows_token_any_kernel<SEPAL_HIP_F16><<<grid, dim3(256), 0, stream>>>(x, ld_x, q, ld_q, scales, ld_s, static_cast<int>(cols)); break;
        }
        check_launch("quantize_rows kernel launch");
        return;
    }
    switch (x_type) {
    case SEPAL_HIP_F32: quant::quantize_rows_token_kernel<SEPAL_HIP_F32><<<grid, dim3(256), 0, stream>>>(x, ld_x, q, ld_q, scales, ld_s, static_cast<int>(cols)); break;
    case SEPAL_HIP_BF16: quant::quantize_rows_token_kernel<SEPAL_HIP_BF16><<<grid, dim3(256), 0, stream>>>(x, ld_x, q, ld_q, scales, ld_s, static_cast<int>(cols)); break;
    default: quant::quantize_rows_token_kernel<SEPAL_HIP_F16><<<grid, dim3(256), 0, stream>>>(x, ld_x, q, ld_q, scales, ld_s, static_cast<int>(cols)); break;
    }
    check_launch("quantize_rows kernel launch");
}

void launch_rmsnorm(const float* x, std::size_t ld_x, void* y, int y_type, std::size_t ld_y, const float* w1,
                    std::size_t rows, std::size_t cols, double eps, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((rows + 3) / 4));  // one row per wave
    const int r = static_cast<int>(rows), c = static_cast<int>(cols);
    using quant::NORM_STORE;
    switch (y_type) {
    case SEPAL_HIP_F32: quant::rmsnorm_kernel<SEPAL_HIP_F32, NORM_STORE><<<grid, dim3(256), 0, stream>>>(x, ld_x, y, ld_y, w1, r, c, eps, nullptr, 0, nullptr, 0); break;
    case SEPAL_HIP_BF16: quant::rmsnorm_kernel<SEPAL_HIP_BF16, NORM_STORE><<<grid, dim3(256), 0, stream>>>(x, ld_x, y, ld_y, w1, r, c, eps, nullptr, 0, nullptr, 0); break;
    default: quant::rmsnorm_kernel<SEPAL_HIP_F16, NORM_STORE><<<grid, dim3(256), 0, stream>>>(x, ld_x, y, ld_y, w1, r, c, eps, nullptr, 0, nullptr, 0); break;
    }
    check_launch("rmsnorm kernel launch");
}

void launch_rmsnorm_quantize(const float* x, std::size_t ld_x, std::uint16_t* y_bf16, std::size_t ld_y, const float* w1,
                             std::int8_t* q, std::size_t ld_q, float* scales, std::size_t ld_s, std::size_t rows,
                             std::size_t cols, std::size_t block, double eps, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
    const int r = static_cast<int>(rows), c = static_cast<int>(cols);
    if (block == 128)
        quant::rmsnorm_kernel<SEPAL_HIP_BF16, quant::NORM_Q_128><<<grid, dim3(256), 0, stream>>>(x, ld_x, y_bf16, ld_y, w1, r, c, eps, q, ld_q, scales, ld_s);
    else
        quant::rmsnorm_kernel<SEPAL_HIP_BF16, quant::NORM_Q_TOKEN><<<grid, dim3(256), 0, stream>>>(x, ld_x, y_bf16, ld_y, w1, r, c, eps, q, ld_q, scales, ld_s);
    check_launch("rmsnorm_quantize kernel launch");
}

void launch_s8_quantize_rows(const void* x, int x_type, std::size_t ld_x, const float* smooth, std::int8_t* q, std::size_t ld_q,
                             float* scales, std::size_t rows, std::size_t cols, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(rows)), block(256);
    const int c = static_cast<int>(cols);
    switch (x_type) {
    case SEPAL_HIP_F32: quant::s8_rows_kernel<SEPAL_HIP_F32><<<grid, block, 0, stream>>>(x, ld_x, smooth, q, ld_q, scales, c); break;
    case SEPAL_HIP_BF16: quant::s8_rows_kernel<SEPAL_HIP_BF16><<<grid, block, 0, stream>>>(x, ld_x, smooth, q, ld_q, scales, c); break;
    default: quant::s8_rows_kernel<SEPAL_HIP_F16><<<grid, block, 0, stream>>>(x, ld_x, smooth, q, ld_q, scales, c); break;
    }
    check_launch("s8 row quantizer launch");
}

void launch_column_stats(const void* x, std::size_t ld_x, std::size_t rows, std::size_t cols, float* amax, double* sums,
                         hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((cols + 255) / 256)), block(256);
    const auto* xp = static_cast<const std::uint16_t*>(x);
    if (sums == nullptr) quant::column_stats_kernel<false><<<grid, block, 0, stream>>>(xp, ld_x, rows, static_cast<int>(cols), amax, nullptr);
    else quant::column_stats_kernel<true><<<grid, block, 0, stream>>>(xp, ld_x, rows, static_cast<int>(cols), amax, sums);
    check_launch("column statistics launch");
}

void launch_broadcast_scales(const float* sw, float* s, std::size_t n, std::size_t groups, hipStream_t stream) {
    quant::broadcast_scales_kernel<<<dim3(static_cast<unsigned>((n * groups + 255) / 256)), dim3(256), 0, stream>>>(sw, s, n, groups);
    check_launch("scale broadcast launch");
}

void launch_f32_to_f16(const float* src, std::size_t ld_src, std::uint16_t* dst, std::size_t ld_dst, std::size_t rows,
                       std::size_t cols, hipStream_t stream) {
    quant::f32_to_f16_kernel<<<dim3(static_cast<unsigned>((rows * cols + 255) / 256)), dim3(256), 0, stream>>>(src, ld_src, dst,
                                                                                                             ld_dst, rows, cols);
    check_launch("float32 to binary16 launch");
}

void launch_f32_to_bf16(const float* src, std::uint16_t* dst, std::size_t count, hipStream_t stream) {
    quant::f32_to_bf16_kernel<<<dim3(static_cast<unsigned>((count + 255) / 256)), dim3(256), 0, stream>>>(src, dst, count);
    check_launch("f32_to_bf16 kernel launch");
}

} // namespace sepal::hip
