// The small-M path (T <= 64 rows) of both multiplies: HBM-bound weight streaming.
//
// At small M every weight byte is used by at most 64 rows, so the multiply is a single pass over the weights and the
// kernel is built to keep HBM busy:
//   - a block (4 waves) owns a column span of 128 weight rows and a range of G groups of k (a split of K); it stages
//     its X slice [16 MT][G x 128] into LDS once, with every load issued before the first store, in rows padded by 16
//     bytes so that the 16 rows an MFMA operand read touches fall in different banks;
//   - each wave owns two 16-column tiles of the span and streams their weights 4 groups at a time: all loads of the
//     next 4-group chunk are issued before the current chunk is multiplied (two register buffers), so a wave keeps
//     up to 2 x 4 x 2 x 16 bytes per lane in flight;
//   - MFMA 16x16x32 (bf16 / binary16, weights widened exactly in registers) or 16x16x64 (int8);
//   - per group: w8g folds the weight scales in Horner form (gemm_w8g.hip), q8 runs the cpu-q8 chain (gemm_q8.hip);
//   - the block's tile goes through LDS; with more than one split the float32 tile is written to the workspace and the
//     last block of the span to arrive (an atomic counter, reset by that block) adds the splits in order and runs the
//     epilogue, so the result does not depend on which block finishes last. With one split the chain is whole and
//     the q8 result equals cpu-q8 bit for bit.
#include <algorithm>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "gemm_kernels.hpp"

namespace sepal::hip {
namespace stream {

enum { KIND_W8G_BF16 = 0, KIND_W8G_F16 = 1, KIND_Q8_GROUP = 2, KIND_Q8_TOKEN = 3 };

constexpr int kSpan = 64;    // weight rows (output columns) per block: one 16-row tile per wave
constexpr int kGMax = 10;    // groups of k one split holds: every weight load of a split is issued at once

template <int KIND>
struct Kind {
    static constexpr bool q8 = KIND >= KIND_Q8_GROUP;
    static constexpr bool per_token = KIND == KIND_Q8_TOKEN;
    static constexpr int xbytes = q8 ? 1 : 2;  // bytes per X element
};

struct Params {
    const void* x;          // [T, ld_x] bf16 / binary16 / int8
    std::size_t ld_x;
    const float* xs;        // q8: activation scales [T, ld_xs]
    std::size_t ld_xs;
    int act_shift;
    const signed char* w;   // [N, ld_w]
    std::size_t ld_w;
    const float* s;         // [N, ld_s]
    std::size_t ld_s;
    void* y;
    std::size_t ld_y;
    int t, n, k;
    int spans, splits, gps;  // column spans, K splits, groups per split
    float* partial;          // [splits][16 MT][spans x 128]
    unsigned* counters;      // [spans]
};

__device__ __forceinline__ f32x4 mfma16_bf16(const u32x4 a, const u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16_f16(const u32x4 a, const u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ i32x4 mfma16_i8(const u32x4 a, const u32x4 b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

// Weight row (output column) of tile column c (0..63) of span `span`. SwiGLU spans take 32 gate rows and the 32 up rows
// of the same features (packed rows 128b + 32h + c and 128b + 64 + 32h + c), so every pair is inside one block.
template <int EP>
__device__ __forceinline__ int span_col(int span, int c) {
    if constexpr (EP == SEPAL_HIP_SWIGLU) {
        const int b = span / 2, h = span % 2;
        return c < 32 ? 128 * b + 32 * h + c : 128 * b + 64 + 32 * h + (c - 32);
    } else {
        return kSpan * span + c;
    }
}

// SILU: 0 the w8g form (HIP's expf / log1pf), 1 the cpu-q8 form (per-128 activation scales), 2 the fast form (q8 with
// one activation scale per token)
template <int EP, int YT, int SILU>
__device__ __forceinline__ void epilogue(const Params& p, const float* tile, int ldt, int rows, int span) {
    // tile [rows][kSpan] floats in LDS; threads write consecutive columns of a row (coalesced)
    if constexpr (EP == SEPAL_HIP_SWIGLU) {
        for (int id = threadIdx.x; id < rows * 32; id += 256) {
            const int r = id / 32, c = id % 32;
            const int f = 64 * (span / 2) + 32 * (span % 2) + c;  // feature of gate row span_col(span, c)
            if (r >= p.t || 2 * f >= p.n) continue;
            const float g = tile[r * ldt + c], u = tile[r * ldt + c + 32];
            store_out<YT>(p.y, static_cast<std::size_t>(r) * p.ld_y + f, SILU == 1 ? swiglu_cephes(g, u) : (SILU == 2 ? swiglu_fast(g, u) : swiglu_libm(g, u)));
        }
    } else {
        float* y = static_cast<float*>(p.y);
        const int n0 = kSpan * span;
        for (int id = threadIdx.x; id < rows * kSpan; id += 256) {
            const int r = id / kSpan, c = id % kSpan;
            if (r >= p.t || n0 + c >= p.n) continue;
            const std::size_t idx = static_cast<std::size_t>(r) * p.ld_y + n0 + c;
            const float v = tile[r * ldt + c];
            y[idx] = EP == SEPAL_HIP_ADD ? __fadd_rn(y[idx], v) : v;
        }
    }
}

template <int KIND, int EP, int YT, int MT>
__global__ void __launch_bounds__(256) gemm_stream(const Params p) {
    using K = Kind<KIND>;
    constexpr int ROWS = 16 * MT;
    extern __shared__ __align__(16) unsigned char lds[];

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int span = blockIdx.x % p.spans, split = blockIdx.x / p.spans;
    const int n0 = span * kSpan;  // this span's columns in the partial-sum layout
    const int groups = p.k / 128;
    const int g0 = split * p.gps, ng = min(p.gps, groups - g0);
    const int xrow = ng * 128 * K::xbytes + 16;  // LDS row stride in bytes (padded)
    float* xs_lds = reinterpret_cast<float*>(lds + ROWS * xrow);  // q8 per-group activation scales [ROWS][ng]

    // ---- every weight load of this wave's tile over the split, issued first ----
    // One 16-row tile per wave; lane l reads row l % 16, 16 bytes at k offset 16 (l / 16) of each 64-k half group.
    // The loads are unconditional (addresses clamped: groups past the split repeat its last group and are never
    // multiplied, columns past N read row 0 and are never stored): a guarded load splits the wave's control flow and
    // the compiler then waits for every load in flight where it joins. Scales are loaded in the same batch, before
    // the weights they scale: the vector memory counter retires loads in order.
    const int col = span_col<EP>(span, wave * 16 + lane % 16);
    const bool col_ok = col < p.n;
    const signed char* wrow = p.w + static_cast<std::size_t>(col_ok ? col : 0) * p.ld_w + g0 * 128 + 16 * (lane / 16);
    const float* srow = p.s + static_cast<std::size_t>(col_ok ? col : 0) * p.ld_s + g0;
    float sc[kGMax];
    u32x4 wb[kGMax][2];
#pragma unroll
    for (int u = 0; u < kGMax; ++u) sc[u] = srow[min(u, ng - 1)];
#pragma unroll
    for (int u = 0; u < kGMax; ++u)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            wb[u][h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + min(u, ng - 1) * 128 + 64 * h));

    // ---- stage X[0..ROWS)[g0*128, +ng*128) into LDS: all loads first, then all stores ----
    {
        const int cpr = ng * 128 * K::xbytes / 16;  // 16-byte chunks per row
        const int total = ROWS * cpr;
        constexpr int MAXC = 4;                       // chunks per thread per batch
        for (int base = 0; base < total; base += 256 * MAXC) {
            u32x4 v[MAXC];
            // unconditional (clamped) loads, as above; rows at or beyond T repeat row T-1 and only feed output rows
            // that are never stored
#pragma unroll
            for (int e = 0; e < MAXC; ++e) {
                const int id = min(base + tid + e * 256, total - 1);
                const int r = min(id / cpr, p.t - 1), c = id % cpr;
                v[e] = *reinterpret_cast<const u32x4*>(static_cast<const unsigned char*>(p.x) +
                                                      (static_cast<std::size_t>(r) * p.ld_x + g0 * 128) * K::xbytes + 16 * c);
            }
#pragma unroll
            for (int e = 0; e < MAXC; ++e) {
                const int id = base + tid + e * 256;
                if (id < total) {
                    const int r = id / cpr, c = id % cpr;
                    *reinterpret_cast<u32x4*>(lds + r * xrow + 16 * c) = v[e];
                }
            }
        }
    }
    if constexpr (K::q8 && !K::per_token) {
        for (int id = tid; id < ROWS * ng; id += 256) {
            const int r = min(id / ng, p.t - 1), gg = id % ng;
            xs_lds[id] = p.xs[static_cast<std::size_t>(r) * p.ld_xs + ((g0 + gg) >> p.act_shift)];
        }
    }
    __syncthreads();

    // ---- multiply ----
    f32x4 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float e = 1.0f, emax = 0.0f;  // the Horner state (the first group's factor multiplies zero accumulators)
    // (all weight loads have landed by now: the X staging above waited for its own loads, which were issued after)
#pragma unroll
    for (int u = 0; u < kGMax; ++u) {
        if (u >= ng) continue;  // fully unrolled: the loaded registers stay registers
        const int kl = u * 128 + 16 * (lane / 16);  // this lane's k offset in the slice (elements)
        if constexpr (!K::q8) {
            // Horner step: rescale the running sum from the previous group's scale to this one; a zero scale marks an
            // all-zero group and keeps e
            const float ratio = horner_step(sc[u], e, emax);
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[i][r] = __fmul_rn(acc[i][r], ratio);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                unsigned o[8];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if constexpr (KIND == KIND_W8G_BF16) s8x4_to_bf16x4(wb[u][h][q], o[2 * q], o[2 * q + 1]);
                    else s8x4_to_f16x4(wb[u][h][q], o[2 * q], o[2 * q + 1]);
                }
                const u32x4 b0 = u32x4{o[0], o[1], o[2], o[3]}, b1 = u32x4{o[4], o[5], o[6], o[7]};
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    const unsigned char* xr = lds + (16 * i + lane % 16) * xrow + (kl + 64 * h) * 2;
                    const u32x4 a0 = *reinterpret_cast<const u32x4*>(xr);
                    const u32x4 a1 = *reinterpret_cast<const u32x4*>(xr + 16);
                    if constexpr (KIND == KIND_W8G_BF16) {
                        acc[i] = mfma16_bf16(a0, b0, acc[i]);
                        acc[i] = mfma16_bf16(a1, b1, acc[i]);
                    } else {
                        acc[i] = mfma16_f16(a0, b0, acc[i]);
                        acc[i] = mfma16_f16(a1, b1, acc[i]);
                    }
                }
            }
        } else {
            // the cpu-q8 chain: y = f_0 * s_0, then fma(f_b, s_b, y); from y = +0 the first fma rounds f_0 * s_0
            // exactly as the product does (float(S) is never -0)
            const i32x4 zero = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const unsigned char* xr = lds + (16 * i + lane % 16) * xrow + kl;
                const u32x4 a0 = *reinterpret_cast<const u32x4*>(xr);
                const u32x4 a1 = *reinterpret_cast<const u32x4*>(xr + 64);
                i32x4 sum = mfma16_i8(a0, wb[u][0], zero);
                sum = mfma16_i8(a1, wb[u][1], sum);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float sc_ = sc[u];
                    if constexpr (!K::per_token) sc_ = __fmul_rn(sc[u], xs_lds[(16 * i + 4 * (lane / 16) + r) * ng + u]);
                    acc[i][r] = __builtin_fmaf(static_cast<float>(sum[r]), sc_, acc[i][r]);
                }
            }
        }
    }

    // ---- the block's tile [ROWS][kSpan] in LDS (over the X slice, which is no longer read) ----
    __syncthreads();
    float* tile = reinterpret_cast<float*>(lds);
    constexpr int ldt = kSpan + 4;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float v = acc[i][r];
            if constexpr (!K::q8) v = __fmul_rn(v, e);
            tile[(16 * i + 4 * (lane / 16) + r) * ldt + wave * 16 + lane % 16] = v;
        }
    __syncthreads();

    if (p.splits > 1) {
        // Hand-off between the blocks of a span without a device-wide fence (on gfx950 one writes back and invalidates
        // the whole L2 of the XCD): the partials are written and read with device-scope relaxed atomics, which go to
        // the device coherence point (global_store/global_load sc1); each thread waits for its stores to complete
        // before the barrier, and only then does one thread count the block in.
        const int npad = p.spans * kSpan;
        for (int id = tid; id < ROWS * kSpan; id += 256) {
            const int r = id / kSpan, c = id % kSpan;
            __hip_atomic_store(&p.partial[(static_cast<std::size_t>(split) * ROWS + r) * npad + n0 + c], tile[r * ldt + c],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        __shared__ unsigned last;
        if (tid == 0)
            last = __hip_atomic_fetch_add(&p.counters[span], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                           static_cast<unsigned>(p.splits - 1) ? 1u : 0u;
        __syncthreads();
        if (last == 0u) return;
        for (int id = tid; id < ROWS * kSpan; id += 256) {
            const int r = id / kSpan, c = id % kSpan;
            const float* src = p.partial + static_cast<std::size_t>(r) * npad + n0 + c;
            const std::size_t step = static_cast<std::size_t>(ROWS) * npad;
            float v = 0.0f;
            for (int s0 = 0; s0 < p.splits; s0 += 8) {  // eight loads in flight, added in split order
                float pv[8];
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    pv[q] = __hip_atomic_load(src + min(s0 + q, p.splits - 1) * step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    if (s0 + q < p.splits) v = s0 + q == 0 ? pv[q] : __fadd_rn(v, pv[q]);
            }
            tile[r * ldt + c] = v;
        }
        if (tid == 0) __hip_atomic_store(&p.counters[span], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
    }
    if constexpr (K::per_token) {
        for (int id = tid; id < ROWS * kSpan; id += 256) {
            const int r = id / kSpan, c = id % kSpan;
            tile[r * ldt + c] = __fmul_rn(tile[r * ldt + c], r < p.t ? p.xs[static_cast<std::size_t>(r) * p.ld_xs] : 0.0f);
        }
        __syncthreads();
    }
    epilogue<EP, YT, K::q8 ? (K::per_token ? 2 : 1) : 0>(p, tile, ldt, ROWS, span);
}

// ---- launch ----------------------------------------------------------------------------------------------------------

// Blocks of a kernel that the device holds at once (occupancy x CUs) with `lds` bytes of dynamic LDS; asked once per
// kernel, device and size.
inline int resident_blocks(const void* kernel, std::size_t lds) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) throw LaunchError("small-M multiply: hipGetDevice failed");
    struct Entry {
        const void* kernel;
        int dev;
        std::size_t lds;
        int blocks;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& e : cache)
        if (e.kernel == kernel && e.dev == dev && e.lds == lds) return e.blocks;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, lds) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        throw LaunchError("small-M multiply: occupancy query failed");
    const int blocks = (per_cu > 0 ? per_cu : 1) * cus;
    cache.push_back({kernel, dev, lds, blocks});
    return blocks;
}

// Groups per split: the fewest splits (fewest partial sums) that still fill the blocks the device holds at once,
// without passing that number (a second round of blocks would wait for the first to drain), at most kGMax groups
// (every weight load of a split is issued at once) and an X slice within 64 KB of LDS.
inline int pick_gps(int spans, int groups, int mt, int xbytes, int force_splits, int resident) {
    const int lds_cap = ((64 << 10) / (16 * mt) - 16) / (128 * xbytes);
    if (force_splits == 1) return groups;  // the caller's LDS check refuses what does not fit
    const int cap = max(1, min(groups, min(lds_cap, kGMax)));
    const int max_splits = max(1, resident / max(1, spans));   // splits that fit in one round
    int gps = (groups + max_splits - 1) / max_splits;          // fewest groups per split within that
    return max(1, min(gps < 1 ? 1 : gps, cap));
}

template <int KIND, int EP, int YT, int MT>
void launch_mt(const GemmArgs& a, hipStream_t stream) {
    using K = Kind<KIND>;
    Params p{};
    p.x = a.x;
    p.ld_x = a.ld_x;
    p.xs = a.xs;
    p.ld_xs = a.ld_xs;
    int shift = 0;
    while ((static_cast<std::size_t>(128) << shift) < a.act_block) ++shift;
    p.act_shift = shift;
    p.w = reinterpret_cast<const signed char*>(a.w);
    p.ld_w = a.ld_w;
    p.s = a.s;
    p.ld_s = a.ld_s;
    p.y = a.y;
    p.ld_y = a.ld_y;
    p.t = static_cast<int>(a.t);
    p.n = static_cast<int>(a.n);
    p.k = static_cast<int>(a.k);
    p.spans = static_cast<int>((a.n + kSpan - 1) / kSpan);
    const int groups = p.k / 128;
    const auto kernel = gemm_stream<KIND, EP, YT, MT>;
    const std::size_t rows = 16 * MT;
    const auto lds_of = [&](int gps) {
        const std::size_t x_bytes = rows * (static_cast<std::size_t>(gps) * 128 * K::xbytes + 16) +
                                    (K::q8 ? rows * gps * sizeof(float) : 0);
        const std::size_t tile_bytes = rows * (kSpan + 4) * sizeof(float);
        return x_bytes > tile_bytes ? x_bytes : tile_bytes;
    };
    // occupancy at the largest slice this instance may take
    const int lds_cap = ((64 << 10) / (16 * MT) - 16) / (128 * K::xbytes);  // as pick_gps
    const int resident = resident_blocks(reinterpret_cast<const void*>(kernel), lds_of(max(1, min(kGMax, min(groups, lds_cap)))));
    p.gps = pick_gps(p.spans, groups, MT, K::xbytes, a.force_splits, resident);
    {
        // no more splits than the workspace's partial zone holds (wide N at 64 rows: 5 MB per split at N = 19456)
        const std::size_t per_split = rows * static_cast<std::size_t>(p.spans) * kSpan * sizeof(float);
        const int max_splits = static_cast<int>(std::max<std::size_t>(1, kPartialBytes / per_split));
        p.gps = max(p.gps, (groups + max_splits - 1) / max_splits);
    }
    p.splits = (groups + p.gps - 1) / p.gps;
    require(a.force_splits != 1 || p.gps <= kGMax, "small-M multiply without a K split (config 2) takes K <= 1280");
    const std::size_t lds = lds_of(p.gps);
    require(lds <= (160u << 10) - 1024, "small-M multiply: K too long for one split (use config 1)");
    if (p.splits > 1) {
        const std::size_t part = static_cast<std::size_t>(p.splits) * rows * p.spans * kSpan * sizeof(float);
        require(static_cast<std::size_t>(p.spans) * sizeof(unsigned) <= kCounterBytes && part <= kPartialBytes,
                "small-M multiply: workspace zone too small for this shape");
        if (a.scratch == nullptr) throw LaunchError("small-M multiply: split-K scratch missing");
        char* ws = static_cast<char*>(a.scratch);
        p.counters = reinterpret_cast<unsigned*>(ws);
        p.partial = reinterpret_cast<float*>(ws + kCounterBytes);
    }
    if (lds > (64u << 10)) {
        raise_dynamic_lds(reinterpret_cast<const void*>(kernel), lds, "small-M multiply");
    }
    kernel<<<dim3(p.spans * p.splits), dim3(256), lds, stream>>>(p);
    check_launch("small-M stream kernel launch");
}

template <int KIND, int EP, int YT>
void launch_rows(const GemmArgs& a, hipStream_t stream) {
    switch ((a.t + 15) / 16) {
    case 1: launch_mt<KIND, EP, YT, 1>(a, stream); break;
    case 2: launch_mt<KIND, EP, YT, 2>(a, stream); break;
    default: launch_mt<KIND, EP, YT, 4>(a, stream); break;
    }
}

template <int KIND>
void launch_ep(const GemmArgs& a, hipStream_t stream) {
    switch (a.epilogue) {
    case SEPAL_HIP_STORE: launch_rows<KIND, SEPAL_HIP_STORE, SEPAL_HIP_F32>(a, stream); break;
    case SEPAL_HIP_ADD: launch_rows<KIND, SEPAL_HIP_ADD, SEPAL_HIP_F32>(a, stream); break;
    default:
        switch (a.y_type) {
        case SEPAL_HIP_F32: launch_rows<KIND, SEPAL_HIP_SWIGLU, SEPAL_HIP_F32>(a, stream); break;
        case SEPAL_HIP_BF16: launch_rows<KIND, SEPAL_HIP_SWIGLU, SEPAL_HIP_BF16>(a, stream); break;
        default: launch_rows<KIND, SEPAL_HIP_SWIGLU, SEPAL_HIP_F16>(a, stream); break;
        }
    }
}

} // namespace stream

void launch_stream_w8g(const GemmArgs& a, hipStream_t stream) {
    if (a.x_type == SEPAL_HIP_BF16) stream::launch_ep<stream::KIND_W8G_BF16>(a, stream);
    else stream::launch_ep<stream::KIND_W8G_F16>(a, stream);
}

void launch_stream_q8(const GemmArgs& a, hipStream_t stream) {
    if (a.act_block == a.k && a.k != 128) stream::launch_ep<stream::KIND_Q8_TOKEN>(a, stream);
    else stream::launch_ep<stream::KIND_Q8_GROUP>(a, stream);
}

} // namespace sepal::hip
