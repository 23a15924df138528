// gpu-q8w on gfx950: int8 activations (one scale per row and 128 values, or per row) times int8 weights (one scale per
// row and 128 values), int32 per-group sums on the int8 MFMA, float32 scale chain over the groups.
//
// Semantics (cpu-q8 I8_Z, runner/src/cpu/gemm_kernels_avx512.cpp:67-115 with finish_tile, gemm.cpp:417-447):
//   S_b = sum over the 128 k of group b of xq * wq            exact int32 (MFMA i32 accumulate)
//   act_block 128:  y = f_0 * (ws_0 * xs_0); y = fma(f_b, ws_b * xs_b, y) for b >= 1, f_b = float(S_b)
//   act_block K:    y = (f_0 * ws_0; y = fma(f_b, ws_b, y)) * xs           (one activation scale per token)
//   epilogue: Store, Add (y + acc), SwiGLU (silu with the cpu-q8 exp polynomial; gate/up rows in the 64-row interleave)
// Every step is one IEEE operation in the reference's order, so the large-M path equals cpu-q8 bit for bit.
//
// Large-M path: 128 x 256 tiles of 8 waves, each 64 x 64 outputs (2 x 2 blocks of MFMA 32x32x32 i8); K in steps of
// one group (128 bytes) through three LDS stages, filled straight from global memory (global_load_lds, whole 128-byte
// rows per 8 lanes) two groups ahead; the int32 sums of a group are turned into the float chain in registers before
// the next group starts (a second set of accumulators holds the chain).
// Small-M path: stream.hip (MFMA 16x16x64 i8; a split of K keeps the sums exact but adds the splits' partial chains in
// split order, within tolerance, not bit for bit).
#include <atomic>

#include "common.hpp"
#include "gemm_kernels.hpp"

namespace sepal::hip {
namespace q8 {

// MODE_CHAIN: the per-group float chain; MODE_SUMS: the int32 group sums out; MODE_WHOLE: one int32 sum over the whole
// K (per-channel weight scales), then (float(S) * sx) * sw (runner/cuda/src/gemm_s8_kernels.cu:255-266); MODE_WHOLE_Y:
// the same sum, then (float(S) * ws) * xs and the chain epilogues (kernel_i8_y, runner/src/cpu/gemm_kernels_avx2.cpp:40-76,
// with finish_tile, gemm.cpp:417-447).
enum { MODE_CHAIN = 0, MODE_SUMS = 1, MODE_WHOLE = 2, MODE_WHOLE_Y = 3 };

__device__ __forceinline__ i32x16 mfma_i8_32(const u32x4 a, const u32x4 b, i32x16 c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}
__device__ __forceinline__ i32x4 mfma_i8_16(const u32x4 a, const u32x4 b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

// One link of the chain: the first group multiplies, later groups fuse.
template <bool PER_TOKEN>
__device__ __forceinline__ float chain(float acc, int sum, float ws, float xs, bool first) {
    const float f = static_cast<float>(sum);
    const float sc = PER_TOKEN ? ws : __fmul_rn(ws, xs);
    return first ? __fmul_rn(f, sc) : __builtin_fmaf(f, sc, acc);
}

template <int EP, int YT>
__device__ __forceinline__ void put(void* y, std::size_t ld_y, int row, int col, float v) {
    float* yf = static_cast<float*>(y);
    const std::size_t idx = static_cast<std::size_t>(row) * ld_y + col;
    if constexpr (EP == SEPAL_HIP_ADD) yf[idx] = __fadd_rn(yf[idx], v);
    else yf[idx] = v;
}

struct Params {
    const signed char* x;   // [T, ld_x]
    std::size_t ld_x;
    const float* xs;        // [T, ld_xs]
    std::size_t ld_xs;
    int act_shift;          // log2(act_block / 128) when per-group; unused per token
    const signed char* w;   // [N, ld_w]
    std::size_t ld_w;
    const float* ws;        // [N, ld_ws]
    std::size_t ld_ws;
    void* y;
    std::size_t ld_y;
    int t, n, k;
    int tiles_m, tiles_n;
    std::int32_t* sums;     // MODE_SUMS: [groups][T][N]
    float* ys;              // kSwigluQ8: [T, ld_ys]
    std::size_t ld_ys;
    // small-M
    int splits, groups_per_split, col_blocks;
    float* partial;
    unsigned* counters;
};

// Logical id of block `bid` among `total`: the hardware places block b on XCD b % 8, and each XCD takes a contiguous
// range of ids, so that consecutive tiles share its L2.
__device__ __forceinline__ int xcd_id(int bid, int total) {
    const int q = total / 8, r = total % 8;
    const int xcd = bid % 8, idx = bid / 8;
    return xcd * q + min(xcd, r) + idx;
}

// Tile of logical id `id`: groups of GM M tiles sweep N with the same few X row panels.
__device__ __forceinline__ void tile_from_id(int id, int tiles_m, int tiles_n, int& tm, int& tn) {
    constexpr int GM = 4;
    const int per_group = GM * tiles_n;
    const int group = id / per_group, first_m = group * GM;
    const int gm = min(tiles_m - first_m, GM);
    const int in_group = id % per_group;
    tm = first_m + in_group % gm;
    tn = in_group / gm;
}

__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
    tile_from_id(xcd_id(bid, tiles_m * tiles_n), tiles_m, tiles_n, tm, tn);
}

// 128-byte LDS rows of 8 chunks; chunk c of row r stored at c ^ ((r / 2) & 7). A 16-byte read is served 16 lanes at a
// time, and a fragment read's 16 lanes take 16 consecutive rows: two rows share a 256-byte bank line, so (r & 1) picks
// the half and (r / 2) & 7 the chunk, and the 16 lanes hit 16 different bank groups (with c ^ (r & 7), rows r and r + 8
// collided: 2-way conflicts on every fragment read).
__device__ __forceinline__ int sw8(int r) { return (r >> 1) & 7; }

// s_waitcnt with the vector memory counter at N and the LDS counter at 0 (gfx9 encoding: vmcnt[3:0] bits 3:0,
// vmcnt[5:4] bits 15:14, expcnt bits 6:4 left at its maximum, lgkmcnt bits 11:8).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));
}

typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void global_void;

// The chain modes' epilogue of a 128 x 256 tile: acc[i][q][r] holds the chain of output (row m0 + wm 64 + 32 i +
// 8 (r / 4) + 4 (lane / 32) + r % 4, column col[q]); per token it is multiplied by the row's activation scale here.
// hb: LDS scratch of 32 KB (kSwigluQ8 only; free when called).
// FAST_SILU: the SwiGLU of the per-token chain (swiglu_q8<true>); the per-128 chain and the AVX2 int8 multiply's
// whole-K form keep the cpu-q8 silu.
template <int EP, int YT, bool PER_TOKEN, bool FAST_SILU = PER_TOKEN>
__device__ __forceinline__ void chain_epilogue(const Params& p, float (&acc)[2][2][16], int m0, int n0, int wm, int ib, int hh,
                                               int lane, int tid, const int (&col)[2], float* hb) {
    constexpr int BM = 128;
    if constexpr (EP == kSwigluQ8) {
        // The tile's 128 output columns are one quantization block. H goes through LDS (the first W stage, free after
        // the loop) in two halves of 64 columns: 128 rows of 256 bytes, 16-byte chunk c of row r at c ^ (r % 16). Thread
        // (row, q) takes 16 columns of one row from each half: the max over them, the four quarters combined through
        // LDS, the scale, and 32 int8 values stored as two 16-byte chunks. max is exact in any order, so this equals
        // quantize_rows on the float32 H (rule RECIPROCAL).
        __shared__ float lds_amax[4][BM];
        const int c = 32 * hh + lane % 32;  // this lane's column within its half (half ib)
        const int row_l = tid % BM, quarter = tid / BM;
        float hv[32];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            if (ib == half) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int rl = wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
                        float v0 = acc[i][0][r], v1 = acc[i][1][r];
                        if constexpr (PER_TOKEN) {
                            const float xs = p.xs[static_cast<std::size_t>(min(m0 + rl, p.t - 1)) * p.ld_xs];
                            v0 = __fmul_rn(v0, xs);
                            v1 = __fmul_rn(v1, xs);
                        }
                        hb[rl * 64 + (((c / 4) ^ (rl % 16)) * 4) + c % 4] = swiglu_q8<FAST_SILU>(v0, v1);
                    }
            }
            __syncthreads();
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v = *reinterpret_cast<const float4*>(hb + row_l * 64 + (((4 * quarter + j) ^ (row_l % 16)) * 4));
                hv[16 * half + 4 * j] = v.x;
                hv[16 * half + 4 * j + 1] = v.y;
                hv[16 * half + 4 * j + 2] = v.z;
                hv[16 * half + 4 * j + 3] = v.w;
            }
            __syncthreads();
        }
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const float a = fabsf(hv[j]);
            m = a > m ? a : m;
        }
        lds_amax[quarter][row_l] = m;
        __syncthreads();
        m = lds_amax[0][row_l];
#pragma unroll
        for (int w = 1; w < 4; ++w) m = lds_amax[w][row_l] > m ? lds_amax[w][row_l] : m;
        const float scale = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
        const float inverse = __fdiv_rn(1.0f, scale);
        const int row = m0 + row_l;
        if (row < p.t) {
            unsigned packed[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                packed[j] = 0u;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float qv = __builtin_rintf(__fmul_rn(hv[4 * j + e], inverse));
                    qv = qv < -127.0f ? -127.0f : (qv > 127.0f ? 127.0f : qv);
                    packed[j] |= (static_cast<unsigned>(static_cast<int>(qv)) & 0xFFu) << (8 * e);
                }
            }
            signed char* dst = static_cast<signed char*>(p.y) + static_cast<std::size_t>(row) * p.ld_y + n0 / 2 + 16 * quarter;
            *reinterpret_cast<u32x4*>(dst) = u32x4{packed[0], packed[1], packed[2], packed[3]};
            *reinterpret_cast<u32x4*>(dst + 64) = u32x4{packed[4], packed[5], packed[6], packed[7]};
            if (quarter == 0) p.ys[static_cast<std::size_t>(row) * p.ld_ys + n0 / 256] = scale;
        }
        return;
    } else {
    // A whole tile needs no bounds checks: the row and the wave's column base are wave-uniform (scalar registers) and
    // the lane adds a 32-bit offset, so a store (and, per token, the row scale's load) costs no vector address
    // arithmetic.
    if (m0 + BM <= p.t && n0 + 256 <= p.n) {
        constexpr unsigned ES = YT == SEPAL_HIP_F32 ? 4 : 2;
        const int wmu = __builtin_amdgcn_readfirstlane(wm), ibu = __builtin_amdgcn_readfirstlane(ib),
                  hhu = __builtin_amdgcn_readfirstlane(hh);
        const unsigned lrow = 4u * static_cast<unsigned>(lane / 32);
        const unsigned voff = (lrow * static_cast<unsigned>(p.ld_y) + lane % 32) * ES;
        const unsigned xoff = lrow * static_cast<unsigned>(p.ld_xs) * 4u;
        char* const yb = static_cast<char*>(p.y);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const std::size_t row = static_cast<std::size_t>(m0 + wmu * 64 + i * 32 + 8 * (r / 4) + (r % 4));
                float v0 = acc[i][0][r], v1 = acc[i][1][r];
                if constexpr (PER_TOKEN) {
                    const float xs = *reinterpret_cast<const float*>(
                        reinterpret_cast<const char*>(p.xs + row * p.ld_xs) + xoff);
                    v0 = __fmul_rn(v0, xs);
                    v1 = __fmul_rn(v1, xs);
                }
                if constexpr (EP == SEPAL_HIP_SWIGLU) {
                    char* const rp = yb + (row * p.ld_y + n0 / 2 + 64 * ibu + 32 * hhu) * ES;
                    store_out<YT>(rp + voff, 0, swiglu_q8<FAST_SILU>(v0, v1));
                } else {
                    // put writes float32
                    const unsigned foff = (lrow * static_cast<unsigned>(p.ld_y) + lane % 32) * 4u;
                    char* const rp0 = yb + (row * p.ld_y + n0 + 128 * ibu + 32 * hhu) * 4;
                    put<EP, YT>(rp0 + foff, 0, 0, 0, v0);
                    put<EP, YT>(rp0 + 256 + foff, 0, 0, 0, v1);
                }
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
            if (row >= p.t) continue;
            float v0 = acc[i][0][r], v1 = acc[i][1][r];
            if constexpr (PER_TOKEN) {
                const float xs = p.xs[static_cast<std::size_t>(row) * p.ld_xs];
                v0 = __fmul_rn(v0, xs);
                v1 = __fmul_rn(v1, xs);
            }
            if constexpr (EP == SEPAL_HIP_SWIGLU) {
                const int f = n0 / 2 + 64 * ib + 32 * hh + lane % 32;
                if (2 * f < p.n) store_out<YT>(p.y, static_cast<std::size_t>(row) * p.ld_y + f, swiglu_q8<FAST_SILU>(v0, v1));
            } else {
                if (col[0] < p.n) put<EP, YT>(p.y, p.ld_y, row, col[0], v0);
                if (col[1] < p.n) put<EP, YT>(p.y, p.ld_y, row, col[1], v1);
            }
        }
    }
    }
}

template <int EP, int YT, bool PER_TOKEN, int MODE>
__global__ void __launch_bounds__(512) gemm_big(const Params p) {
    constexpr int BM = 128, BN = 256;
    constexpr int XDMA = BM / 64, WDMA = BN / 64;  // direct loads per thread and group (8 rows of 128 bytes each)
    constexpr int NSC = MODE == MODE_CHAIN ? (PER_TOKEN ? 2 : 3) : 0;  // scale loads per thread and group
    constexpr bool WHOLE = MODE == MODE_WHOLE || MODE == MODE_WHOLE_Y;
    // Three stages of each operand, each its own LDS array: the compiler then knows which array a direct load writes,
    // and a fragment read waits only for loads into the array it reads.
    __shared__ __align__(1024) u32x4 lx0[BM * 8], lx1[BM * 8], lx2[BM * 8];
    __shared__ __align__(1024) u32x4 lw0[BN * 8], lw1[BN * 8], lw2[BN * 8];
    __shared__ float lds_xs[2][BM];
    const auto xstage = [&](auto it) -> u32x4* {
        constexpr int i = decltype(it)::value;
        if constexpr (i == 0) return lx0;
        else if constexpr (i == 1) return lx1;
        else return lx2;
    };
    const auto wstage = [&](auto it) -> u32x4* {
        constexpr int i = decltype(it)::value;
        if constexpr (i == 0) return lw0;
        else if constexpr (i == 1) return lw1;
        else return lw2;
    };

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int wm = wave % 2, wn = wave / 2;
    int tm, tn;
    tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int groups = p.k / 128;

    // ---- direct loads: load e of wave w fills LDS kilobyte w + 8 e = rows 8 w + 64 e + {0..7} of the stage; lane l
    // writes slot l % 8 of row 8 w + 64 e + l / 8, which holds chunk (l % 8) ^ sw8(row) = (l % 8) ^ ((4 w + l / 16) & 7).
    // Sources are clamped: rows past T or N repeat the last row; their outputs are never stored.
    const int chunk = (lane % 8) ^ ((4 * wave + lane / 16) & 7);
    const signed char* xsrc[XDMA];
    const signed char* wsrc[WDMA];
#pragma unroll
    for (int e = 0; e < XDMA; ++e)
        xsrc[e] = p.x + static_cast<std::size_t>(min(m0 + 8 * wave + 64 * e + lane / 8, p.t - 1)) * p.ld_x + 16 * chunk;
#pragma unroll
    for (int e = 0; e < WDMA; ++e)
        wsrc[e] = p.w + static_cast<std::size_t>(min(n0 + 8 * wave + 64 * e + lane / 8, p.n - 1)) * p.ld_w + 16 * chunk;
    const float* xs_row = p.xs + static_cast<std::size_t>(min(m0 + (tid % BM), p.t - 1)) * p.ld_xs;

    const int ib = wn / 2, hh = wn % 2;
    const int colrel[2] = {128 * ib + 32 * hh + lane % 32, 128 * ib + 64 + 32 * hh + lane % 32};
    int col[2];
    const float* wsrow[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        col[j] = n0 + colrel[j];
        wsrow[j] = p.ws + static_cast<std::size_t>(min(col[j], p.n - 1)) * p.ld_ws;
    }

    // one group's scales, in registers; three sets rotate with the stages (group g's in set g mod 3)
    struct Set {
        float xs, ws[2];
    };
    const auto issue = [&](int g, u32x4* xd, u32x4* wd, Set& s) {
        const std::size_t k0 = static_cast<std::size_t>(g) * 128;
#pragma unroll
        for (int e = 0; e < XDMA; ++e)
            __builtin_amdgcn_global_load_lds((global_void*)(xsrc[e] + k0), (lds_void*)(xd + (wave + 8 * e) * 64), 16, 0, 0);
#pragma unroll
        for (int e = 0; e < WDMA; ++e)
            __builtin_amdgcn_global_load_lds((global_void*)(wsrc[e] + k0), (lds_void*)(wd + (wave + 8 * e) * 64), 16, 0, 0);
        if constexpr (!PER_TOKEN && MODE == MODE_CHAIN) s.xs = xs_row[g >> p.act_shift];
        if constexpr (MODE == MODE_CHAIN) {
            s.ws[0] = wsrow[0][g];
            s.ws[1] = wsrow[1][g];
        }
    };
    // per-128 activation scales of the next group into their LDS buffer
    const auto stage_xs = [&](int buf, const Set& s) {
        if constexpr (!PER_TOKEN && MODE == MODE_CHAIN)
            if (tid < BM) lds_xs[buf][tid] = s.xs;
    };
    // the wait leaves the loads issued by the current step in flight and covers every earlier one, among them the next
    // group's operands; a workgroup release fence would also wait for the loads two groups ahead
    const auto barrier = [&]() {
        asm volatile("" ::: "memory");
        wait_vm_lgkm0<XDMA + WDMA + NSC>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    float acc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    const i32x16 zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    i32x16 tot[2][2] = {{zero16, zero16}, {zero16, zero16}};  // MODE_WHOLE: the running int32 sums

    // Group g (j = g mod 3): issue group g + 2's loads (clamped) into stage (j + 2) mod 3, last read by group g - 1; the
    // exact int32 sums of group g from stage j; its link of the scale chain (or the sums out); group g + 1's per-128
    // activation scales into LDS; one barrier. The loads are issued at every step, past the last group too (repeats
    // into stages nothing reads again), so the wait count of the barrier stays exact.
    Set s0, s1, s2;
    const auto step = [&](int g, auto jt, auto first_t) {
        constexpr int j = decltype(jt)::value;
        constexpr bool first = decltype(first_t)::value;  // group 0: its link multiplies (known at compile time)
        Set& cur = j == 0 ? s0 : (j == 1 ? s1 : s2);
        Set& next = j == 0 ? s1 : (j == 1 ? s2 : s0);
        Set& free_ = j == 0 ? s2 : (j == 1 ? s0 : s1);
        issue(min(g + 2, groups - 1), xstage(std::integral_constant<int, (j + 2) % 3>{}),
              wstage(std::integral_constant<int, (j + 2) % 3>{}), free_);
        __builtin_amdgcn_sched_barrier(0);
        if (g < groups) {
            const int buf = g & 1;
            const u32x4* tx = xstage(std::integral_constant<int, j>{});
            const u32x4* tw = wstage(std::integral_constant<int, j>{});
            i32x16 sacc[2][2];
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const int c = 2 * st + lane / 32;
                u32x4 a[2], b[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int row = wm * 64 + i * 32 + lane % 32;
                    a[i] = tx[row * 8 + (c ^ sw8(row))];
                }
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int row = colrel[q];
                    b[q] = tw[row * 8 + (c ^ sw8(row))];
                }
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        if constexpr (WHOLE) tot[i][q] = mfma_i8_32(a[i], b[q], tot[i][q]);
                        else sacc[i][q] = mfma_i8_32(a[i], b[q], st == 0 ? zero16 : sacc[i][q]);
                    }
            }
            if constexpr (WHOLE) {
            } else if constexpr (MODE == MODE_SUMS) {
                // the row base is opaque here, so that the 64 store addresses are not hoisted out of the loop (spills)
                int mb = m0;
                asm volatile("" : "+s"(mb));
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = mb + wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
                        if (row >= p.t) continue;
#pragma unroll
                        for (int q = 0; q < 2; ++q)
                            if (col[q] < p.n) p.sums[(static_cast<std::size_t>(g) * p.t + row) * p.n + col[q]] = sacc[i][q][r];
                    }
            } else {
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int rl = wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
                        const float xsv = PER_TOKEN ? 1.0f : lds_xs[buf][rl];
#pragma unroll
                        for (int q = 0; q < 2; ++q) acc[i][q][r] = chain<PER_TOKEN>(acc[i][q][r], sacc[i][q][r], cur.ws[q], xsv, first);
                    }
            }
            if (g + 1 < groups) stage_xs(buf ^ 1, next);
        }
        barrier();
    };

    // the whole-K modes take K a multiple of 16: whole groups here, the rest (tail) after the loop
    if (groups > 0) {
    issue(0, lx0, lw0, s0);
    issue(min(1, groups - 1), lx1, lw1, s1);
    __builtin_amdgcn_sched_barrier(0);
    stage_xs(0, s0);
    asm volatile("" ::: "memory");
    wait_vm_lgkm0<XDMA + WDMA + NSC>();  // group 0's loads
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // group 0 on its own (its link of the chain multiplies), then three groups per iteration (stage g mod 3)
    step(0, std::integral_constant<int, 0>{}, std::true_type{});
    for (int g = 1; g < groups; g += 3) {
        step(g, std::integral_constant<int, 1>{}, std::false_type{});
        step(g + 1, std::integral_constant<int, 2>{}, std::false_type{});
        step(g + 2, std::integral_constant<int, 0>{}, std::false_type{});
    }
    // the repeated loads of the last steps may still be writing LDS: drain them before the block reuses or leaves it
    wait_vm_lgkm0<0>();
    __syncthreads();
    }
    if constexpr (WHOLE) {
        // the last K % 128 values (a multiple of 16): each lane loads its fragment chunks straight from global memory
        // (rows clamped as above, chunks at or past K read as zero) and the MFMAs add them to the int32 sums
        const int k0 = groups * 128, tail = p.k - k0;
        if (tail > 0) {
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                if (32 * st >= tail) break;
                const int c = 2 * st + lane / 32;
                const bool in = 16 * c < tail;
                u32x4 a[2], b[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int row = min(m0 + wm * 64 + i * 32 + lane % 32, p.t - 1);
                    a[i] = in ? *reinterpret_cast<const u32x4*>(p.x + static_cast<std::size_t>(row) * p.ld_x + k0 + 16 * c)
                              : u32x4{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int row = min(n0 + colrel[q], p.n - 1);
                    b[q] = in ? *reinterpret_cast<const u32x4*>(p.w + static_cast<std::size_t>(row) * p.ld_w + k0 + 16 * c)
                              : u32x4{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int q = 0; q < 2; ++q) tot[i][q] = mfma_i8_32(a[i], b[q], tot[i][q]);
            }
        }
    }
    if constexpr (MODE == MODE_SUMS) return;
    if constexpr (MODE == MODE_WHOLE) {
        // y = (float(S) * sx[t]) * sw[n], float32 or binary16 (round to nearest even)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
                if (row >= p.t) continue;
                const float sx = p.xs[static_cast<std::size_t>(row) * p.ld_xs];
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    if (col[j] < p.n) {
                        const float v = __fmul_rn(__fmul_rn(static_cast<float>(tot[i][j][r]), sx), wsrow[j][0]);
                        const std::size_t idx = static_cast<std::size_t>(row) * p.ld_y + col[j];
                        if constexpr (YT == SEPAL_HIP_F16) static_cast<unsigned short*>(p.y)[idx] = f32_to_f16_bits(v);
                        else static_cast<float*>(p.y)[idx] = v;
                    }
            }
        return;
    }
    if constexpr (MODE == MODE_WHOLE_Y) {
        // float(S) * ws[n]; the per-token epilogue multiplies by xs[t]
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = __fmul_rn(static_cast<float>(tot[i][j][r]), wsrow[j][0]);
    }

    chain_epilogue<EP, YT, PER_TOKEN, PER_TOKEN && MODE == MODE_CHAIN>(p, acc, m0, n0, wm, ib, hh, lane, tid, col, reinterpret_cast<float*>(lw0));
}

// ---- the chain, two wave groups in alternation (gemm_chain) ---------------------------------------------------------
//
// The 128 x 256 tile of gemm_big's chain mode: 8 waves of 64 x 64 outputs (2 x 2 blocks of MFMA 32x32x32 i8), K in
// steps of one group (128 bytes) through three LDS stages of 128-byte rows (chunk c of row r at c ^ sw8(r)), filled
// straight from global memory through buffer descriptors (a 32-bit lane offset: the row, clamped to the last row, and
// the swizzled chunk; the group's offset in the scalar offset; the LDS destination in scalar registers). Each block's
// four MFMAs give its exact int32 group sums, and the cpu-q8 chain links them into the float accumulators
// (per token acc = f_0 ws_0, then acc = fma(f_g, ws_g, acc), times the token's scale in the epilogue; per 128 the
// scale of a link is ws_g x xs_g of the output's row, from an LDS ring of the tile rows' scales), each output's links in
// group order, so the results do not depend on how the work is scheduled.
// Schedule: waves 0-3 (group A, one per SIMD) and 4-7 (group B) each alternate two slots per group, separated by
// block barriers, so that in every slot one wave of each SIMD reads the LDS while the other runs MFMAs and the chain's
// VALU work (with every wave reading after the same barrier and then multiplying, the two waves of a SIMD waited for
// the LDS together and then competed for the MFMA and VALU units together: 8% slower at C4). L(g) issues the wave's
// share of group g + 2's direct loads (2 of the activations' and 4 of the weights' 1 KB loads, and its two weight
// scales) into the stage of group g - 1 and reads all 16 operand fragments of group g; M(g) runs the group's four
// blocks, each block's MFMAs with the link of the block LAG before it (two per token, whose sums were complete a block
// ago; one per 128, issued after the block's own MFMAs), so the link's converts and fused multiply-adds interleave with
// the MFMAs. Group B runs one slot behind group A: slot 2g is
// A L(g) and B M(g - 1), slot 2g + 1 is A M(g) and B L(g). Stage g mod 3 is last read in slot 2g + 1 and reloaded
// (with group g + 3) from slot 2g + 2. At the end of L(g) a wave waits for its share of group g + 1 (issued in its
// previous L slot), so both shares are complete by the barrier that ends slot 2g + 1, before group g + 1 is first
// read; every wave issues, reads and waits alike (only B's extra barrier at the start and A's at the end differ), so
// the kernel has no branch between the groups' code. The launcher uses this kernel when every offset fits 32 bits.
struct ChainParams {
    Params p;
    unsigned x_bytes, w_bytes, ws_bytes, xs_bytes;  // extents of X, W and their scales (buffer ranges)
};

template <int EP, int YT, bool PER_TOKEN>
__global__ void __launch_bounds__(512) gemm_chain(const ChainParams cp) {
    const Params& p = cp.p;
    constexpr int BM = 128, BN = 256;
    // a wave's loads per group: its operand shares, its 2 weight scales and, per 128, one activation scale
    constexpr int XDMA = BM / 64, WDMA = BN / 64, NLD = XDMA + WDMA + 2 + (PER_TOKEN ? 0 : 1);
    __shared__ __align__(1024) u32x4 lx0[BM * 8], lx1[BM * 8], lx2[BM * 8];
    __shared__ __align__(1024) u32x4 lw0[BN * 8], lw1[BN * 8], lw2[BN * 8];
    // per 128: the tile rows' activation scales of group g in ring slot (xb + g) mod 4. Four slots, not three: group
    // B's M slot of group g reads the scales of groups g and g - 1 in the slot where group A writes those of group
    // g + 2 (xb carries the ring on from tile to tile, so a tile's first write never meets the previous tile's last
    // links)
    __shared__ __align__(16) float lds_xs[4][BM];
    typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
    const auto xstage = [&](auto it) -> lds_u32x4* {
        constexpr int i = decltype(it)::value;
        if constexpr (i == 0) return (lds_u32x4*)lx0;
        else if constexpr (i == 1) return (lds_u32x4*)lx1;
        else return (lds_u32x4*)lx2;
    };
    const auto wstage = [&](auto it) -> lds_u32x4* {
        constexpr int i = decltype(it)::value;
        if constexpr (i == 0) return (lds_u32x4*)lw0;
        else if constexpr (i == 1) return (lds_u32x4*)lw1;
        else return (lds_u32x4*)lw2;
    };

    const int tid = threadIdx.x, lane = tid % 64;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);  // wave-uniform: LDS destinations stay scalar
    const bool group_b = wave >= 4;
    const int wm = wave % 2, wn = wave / 2;
    // persistent: one block per CU; block b works through the contiguous range [lo, hi) of logical tiles of its XCD
    // (b mod 8), every (gridDim.x / 8)-th from lo + b / 8, so the XCD's blocks run consecutive tiles at a time (they
    // share its L2)
    const int total = p.tiles_m * p.tiles_n;
    int cur, hi, stride;
    {
        const int nx = static_cast<int>(gridDim.x) / 8, xcd = static_cast<int>(blockIdx.x) % 8;
        const int q = total / 8, r = total % 8;
        const int lo = xcd * q + min(xcd, r);
        hi = lo + q + (xcd < r ? 1 : 0);
        cur = lo + static_cast<int>(blockIdx.x) / 8;
        stride = nx;
    }
    if (cur >= hi || stride < 1) return;  // (the launcher's grid is a positive multiple of 8, so stride >= 1)
    const int groups = p.k / 128;

    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(const_cast<signed char*>(p.x), 0, static_cast<int>(cp.x_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(const_cast<signed char*>(p.w), 0, static_cast<int>(cp.w_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t wsres = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.ws), 0, static_cast<int>(cp.ws_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t xsres = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.xs), 0, static_cast<int>(cp.xs_bytes), 0x00020000);
    // a wave's share of a group's loads: direct load e fills LDS kilobyte wave + 8 e = rows 8 wave + 64 e + {0..7};
    // lane l writes slot l % 8 of row 8 wave + 64 e + l / 8, which holds chunk (l % 8) ^ sw8(row) = (l % 8) ^
    // ((4 wave + l / 16) & 7); rows past T or N repeat the last row (never stored)
    const int chunk = (lane % 8) ^ ((4 * wave + lane / 16) & 7);
    const int ib = wn / 2, hh = wn % 2;
    const int colrel[2] = {128 * ib + 32 * hh + lane % 32, 128 * ib + 64 + 32 * hh + lane % 32};
    // the tile's origin and the offsets that depend on it
    int m0, n0, xoff[XDMA], woff[WDMA], ws_off0, ws_off1, xs_off;
    const auto set_tile = [&]() __attribute__((always_inline)) {
        int tm, tn;
        tile_from_id(cur, p.tiles_m, p.tiles_n, tm, tn);
        m0 = tm * BM;
        n0 = tn * BN;
#pragma unroll
        for (int e = 0; e < XDMA; ++e)
            xoff[e] = min(m0 + 8 * wave + 64 * e + lane / 8, p.t - 1) * static_cast<int>(p.ld_x) + 16 * chunk;
#pragma unroll
        for (int e = 0; e < WDMA; ++e)
            woff[e] = min(n0 + 8 * wave + 64 * e + lane / 8, p.n - 1) * static_cast<int>(p.ld_w) + 16 * chunk;
        ws_off0 = min(n0 + colrel[0], p.n - 1) * static_cast<int>(p.ld_ws) * 4;
        ws_off1 = min(n0 + colrel[1], p.n - 1) * static_cast<int>(p.ld_ws) * 4;
        // per 128: lane l % 16 of wave w loads the scale of tile row 16 w + l % 16 (clamped like the operands)
        xs_off = min(m0 + 16 * wave + lane % 16, p.t - 1) * static_cast<int>(p.ld_xs) * 4;
    };
    set_tile();
    int ra[4], rb[4];
    {
        const int rowa = wm * 64 + lane % 32, rowb = colrel[0];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const int c = 2 * st + lane / 32;
            ra[st] = rowa * 8 + (c ^ sw8(rowa));
            rb[st] = rowb * 8 + (c ^ sw8(rowb));
        }
    }

    struct Set {
        float ws[2];
        float xs;  // per 128: the activation scale of this lane's staging row
    };
    Set s0, s1, s2;  // group g's scales in set g mod 3
    // the wave's loads of group g: its share of one operand's stage, then its two weight scales
    const auto issue = [&](int g, lds_u32x4* xd, lds_u32x4* wd, Set& s) {
        const int k0 = g * 128;
#pragma unroll
        for (int e = 0; e < XDMA; ++e)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (__attribute__((address_space(3))) void*)(xd + (wave + 8 * e) * 64), 16,
                                                     xoff[e], k0, 0, 0);
#pragma unroll
        for (int e = 0; e < WDMA; ++e)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wres, (__attribute__((address_space(3))) void*)(wd + (wave + 8 * e) * 64), 16,
                                                     woff[e], k0, 0, 0);
        s.ws[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wsres, ws_off0, g * 4, 0));
        s.ws[1] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wsres, ws_off1, g * 4, 0));
        if constexpr (!PER_TOKEN)
            s.xs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xsres, xs_off, (g >> p.act_shift) * 4, 0));
    };
    int xb = 0;  // ring slot of the current tile's group 0
    // per 128: group g's scales (landed) from set s into their ring slot; the LDS write is complete on return
    const auto put_xs = [&](int g, const Set& s) __attribute__((always_inline)) {
        if constexpr (!PER_TOKEN) {
            // every lane writes (lanes l, l + 16, l + 32, l + 48 the same value): no branch, which costs the kernel its
            // registers
            lds_xs[(xb + g) & 3][16 * wave + lane % 16] = s.xs;
            wait_vm_lgkm0<NLD>();
        }
    };
    const auto barrier = [&]() __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };

    float acc[2][2][16];
    const i32x16 zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    // int32 sums of the blocks in flight: block n = 4 g + b (group g, block b) in T[n mod 3] (with three groups a turn
    // the index is a constant: (4 (g mod 3) + b) mod 3)
    // Per 128 the links run one block behind (two buffers, index n mod 2): each link also reads 16 activation scales,
    // and beside a third buffer's 16 registers the SwiGLU -> int8 form spilled 44 registers and took 1.77 against
    // 1.52 ms at C4's gate/up (the down multiply ran alike both ways). The block's four MFMAs are issued before its
    // link, so the converts still find the previous block's sums complete.
    constexpr int NT = PER_TOKEN ? 3 : 2, LAG = NT - 1;
    i32x16 T[NT];
    u32x4 a[2][4], b[2][4];
    // one link: per token acc = f ws (first group) or fma(f, ws, acc); per 128 the scale is ws x xs of the output's
    // row in group g (the cpu-q8 chain, as gemm_big's)
    const auto link = [&](const i32x16& S, int i, int q, float ws, bool first, int g) {
        if constexpr (PER_TOKEN) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float f = static_cast<float>(S[r]);
                acc[i][q][r] = first ? __fmul_rn(f, ws) : __builtin_fmaf(f, ws, acc[i][q][r]);
            }
        } else {
            const float* xr = lds_xs[(xb + g) & 3] + wm * 64 + i * 32 + 4 * (lane / 32);
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const float4 x4 = *reinterpret_cast<const float4*>(xr + 8 * r4);
                const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * r4 + e;
                    const float f = static_cast<float>(S[r]);
                    const float sc = __fmul_rn(ws, xv[e]);
                    acc[i][q][r] = first ? __fmul_rn(f, sc) : __builtin_fmaf(f, sc, acc[i][q][r]);
                }
            }
        }
    };

    // L(g), stage j = g mod 3: group g + 2's loads (clamped: past the end they repeat into stages nothing reads again,
    // so the wait counts stay exact) into the stage and scale set of group g - 1, then group g's 16 fragments; the
    // reads are complete before the barrier
    const auto slot_l = [&](int g, auto jt) __attribute__((always_inline)) {
        constexpr int j = decltype(jt)::value;
        Set& nxt = j == 0 ? s2 : (j == 1 ? s0 : s1);
        const Set& following = j == 0 ? s1 : (j == 1 ? s2 : s0);  // group g + 1's
        issue(min(g + 2, groups - 1), xstage(std::integral_constant<int, (j + 2) % 3>{}),
              wstage(std::integral_constant<int, (j + 2) % 3>{}), nxt);
        __builtin_amdgcn_sched_barrier(0);
        const lds_u32x4* tx = xstage(std::integral_constant<int, j>{});
        const lds_u32x4* tw = wstage(std::integral_constant<int, j>{});
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            a[0][st] = tx[ra[st]];
            b[0][st] = tw[rb[st]];
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            a[1][st] = tx[ra[st] + 256];
            b[1][st] = tw[rb[st] + 512];
        }
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        wait_vm_lgkm0<NLD>();  // and the wave's loads of group g + 1 (its loads of group g + 2 stay in flight)
        // (unconditional, as a branch here also costs registers: past the last group the write puts the clamped repeat
        // into the slot of the next tile's group 0, which held group groups - 4, read by no slot still running; the next
        // tile writes that slot again after the barriers that end this tile)
        put_xs(g + 1, following);
        barrier();
    };
    // M(g): blocks 0..3, each block's four MFMAs with the link of the block LAG before it (the last LAG blocks of group
    // g - 1 at the first LAG blocks), so the link's converts and fused multiply-adds interleave with the MFMAs instead
    // of waiting for the last one; every output's links still run in group order. The last group's last LAG blocks are
    // linked after its M slot.
    float pw0 = 0.0f, pw1 = 0.0f;  // group g - 1's weight scales
    const auto slot_m = [&](int g, auto jt, auto prev_t) __attribute__((always_inline)) {
        constexpr int j = decltype(jt)::value;
        // 0: group 0 (no previous group; its own links multiply); 1: group 1 (group 0's last blocks link by a
        // multiply); 2: later groups
        constexpr int pmode = decltype(prev_t)::value;
        constexpr bool first = pmode == 0;
        Set& cur = j == 0 ? s0 : (j == 1 ? s1 : s2);
        const float gws0 = cur.ws[0], gws1 = cur.ws[1];
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
            const int i = blk / 2, q = blk % 2;
            i32x16& S = T[(4 * j + blk) % NT];
#pragma unroll
            for (int st = 0; st < 4; ++st) S = mfma_i8_32(a[i][st], b[q][st], st == 0 ? zero16 : S);
            if (blk >= LAG) {
                const int pb = blk - LAG;  // this group's block pb
                link(T[(4 * j + pb) % NT], pb / 2, pb % 2, pb % 2 == 0 ? gws0 : gws1, first, g);
            } else if constexpr (pmode > 0) {
                const int pb = blk + 4 - LAG;  // the previous group's block pb
                link(T[(4 * j + blk + NT - LAG) % NT], pb / 2, pb % 2, pb % 2 == 0 ? pw0 : pw1, pmode == 1, g - 1);
            }
        }
        pw0 = gws0;
        pw1 = gws1;
        barrier();
    };

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    // a tile's first loads: groups 0 and 1 in stages and scale sets 0 and 1
    const auto first_loads = [&]() __attribute__((always_inline)) {
        issue(0, xstage(I0{}), wstage(I0{}), s0);
        issue(min(1, groups - 1), xstage(I1{}), wstage(I1{}), s1);
    };
    first_loads();
    // Tile loop. Per tile the barriers balance (group A: 1 + 2 groups + 1, group B: 1 + 1 + 2 groups); after the last
    // one every wave has read the tile's stages for the last time, so once a wave has waited for its own loads (the
    // clamped repeats of the last groups) it issues the next tile's first loads, which fly while this tile's epilogue
    // runs (its outputs go straight to global memory). The SwiGLU -> int8 epilogue uses weight stage 0 as scratch, so
    // there the next tile's loads follow it.
    for (;;) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        wait_vm_lgkm0<NLD>();  // group 0's loads
        put_xs(0, s0);
        barrier();
        if (group_b) barrier();  // B runs one slot behind A
        // group g in stage and scale set g mod 3; M of group 0 and group 1 by their own modes, then three groups a turn
        slot_l(0, I0{});
        slot_m(0, I0{}, I0{});
        int g = 1;
        if (groups > 1) {
            slot_l(1, I1{});
            slot_m(1, I1{}, I1{});
            g = 2;
        }
        for (; g + 3 <= groups; g += 3) {
            slot_l(g, I2{});
            slot_m(g, I2{}, I2{});
            slot_l(g + 1, I0{});
            slot_m(g + 1, I0{}, I2{});
            slot_l(g + 2, I1{});
            slot_m(g + 2, I1{}, I2{});
        }
        if (g < groups) {
            slot_l(g, I2{});
            slot_m(g, I2{}, I2{});
        }
        if (g + 1 < groups) {
            slot_l(g + 1, I0{});
            slot_m(g + 1, I0{}, I2{});
        }
        if (!group_b) barrier();  // matches group B's extra barrier
        // the last group's last LAG blocks (group groups - 1, stage index (groups - 1) mod 3)
        const auto last_links = [&](auto jt) __attribute__((always_inline)) {
            constexpr int j = decltype(jt)::value;
#pragma unroll
            for (int pb = 4 - LAG; pb < 4; ++pb)
                link(T[(4 * j + pb) % NT], pb / 2, pb % 2, pb % 2 == 0 ? pw0 : pw1, groups == 1, groups - 1);
        };
        switch ((groups - 1) % 3) {
        case 0: last_links(I0{}); break;
        case 1: last_links(I1{}); break;
        default: last_links(I2{}); break;
        }
        wait_vm_lgkm0<0>();  // this wave's repeated loads of the last groups have landed
        const int mc = m0, nc = n0;
        const int col[2] = {nc + colrel[0], nc + colrel[1]};
        cur += stride;
        const bool more = cur < hi;
        xb = (xb + groups) & 3;  // the next tile's group 0 takes the ring slot after this tile's last group
        if constexpr (EP == kSwigluQ8) {
            __syncthreads();
            chain_epilogue<EP, YT, PER_TOKEN>(p, acc, mc, nc, wm, ib, hh, lane, tid, col, reinterpret_cast<float*>(lw0));
            __syncthreads();  // weight stage 0 (the epilogue's scratch) is free again
            if (!more) break;
            set_tile();
            first_loads();
        } else {
            if (more) {
                set_tile();
                first_loads();
            }
            chain_epilogue<EP, YT, PER_TOKEN>(p, acc, mc, nc, wm, ib, hh, lane, tid, col, reinterpret_cast<float*>(lw0));
            if (!more) break;
        }
    }
}

// ---- gemm_s8 (per-channel W8A8, int32 sums over the whole K): 256 x 256 tiles ----------------------------------------
//
// 8 waves of 128 x 64 outputs (4 x 2 blocks of MFMA 32x32x32 i8, 128 int32 accumulators), K in steps of 64 bytes. Both
// operands go straight from global memory into LDS (buffer_load ... lds, 16 bytes a lane, 16 rows x 64 bytes per
// instruction), row-major with 64-byte rows, chunk c of row r at slot c ^ ((r / 4) & 3): every 16 lanes of a fragment
// read (16 rows, one chunk) cover the 16 bank groups. Three stages of each, separate LDS arrays (the compiler then
// knows which array a direct load writes); the loads of step kt + 2 are issued while step kt is multiplied, and each
// step ends with an explicit wait and a bare barrier. MB 2 gives 128 x 256 halves for a launch's last partial round.
// The sums are exact, so the results equal gemm_big's whole-K mode bit for bit.
struct S8Params {
    const signed char* x;
    std::size_t ld_x;
    const float* xs;
    std::size_t ld_xs;
    const signed char* w;
    std::size_t ld_w;
    const float* ws;
    std::size_t ld_ws;
    void* y;
    std::size_t ld_y;
    int t, n, k;
    int tiles_m, tiles_n, id0, count;
    std::size_t x_bytes, w_bytes;
};

template <int YT, int MB>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) gemm_s8_big(const S8Params p) {
    constexpr int NW = 8, KS = 64, SUB = KS / 32, BM = 64 * MB, BN = 256;
    constexpr int XSTAGE = BM * KS, WSTAGE = BN * KS;
    constexpr int XLD = XSTAGE / 1024 / NW, WLD = WSTAGE / 1024 / NW;  // 1 KB direct loads per wave and step
    __shared__ __align__(1024) unsigned char xs0[XSTAGE], xs1[XSTAGE], xs2[XSTAGE], ws0[WSTAGE], ws1[WSTAGE], ws2[WSTAGE];
    const auto xstage = [&](auto it) -> unsigned char* {
        constexpr int i = decltype(it)::value;
        if constexpr (i == 0) return xs0;
        else if constexpr (i == 1) return xs1;
        else return xs2;
    };
    const auto wstage = [&](auto it) -> unsigned char* {
        constexpr int i = decltype(it)::value;
        if constexpr (i == 0) return ws0;
        else if constexpr (i == 1) return ws1;
        else return ws2;
    };

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int wm = wave % 2, wn = wave / 2;
    int tm, tn, m0;
    if constexpr (MB == 4) {
        tile_from_id(p.id0 + xcd_id(blockIdx.x, p.count), p.tiles_m, p.tiles_n, tm, tn);
        m0 = tm * 256;
    } else {
        const int b = blockIdx.x;
        tile_from_id(p.id0 + b % p.count, p.tiles_m, p.tiles_n, tm, tn);
        m0 = tm * 256 + (b / p.count) * BM;
    }
    const int n0 = tn * BN;
    const int KT = p.k / KS;

    // rows past T or N read as zero (past num_records); the launcher checks that every offset fits 32 bits
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<signed char*>(p.x), 0, static_cast<int>(p.x_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<signed char*>(p.w), 0, static_cast<int>(p.w_bytes), 0x00020000);
    // direct load i of wave w fills LDS kilobyte w + 8 i = rows 16 w + 128 i + {0..15}; lane l writes slot l % 4 of row
    // 16 w + 128 i + l / 4, which holds chunk (l % 4) ^ ((row / 4) & 3) = (l % 4) ^ ((l / 16) & 3)
    const int lrow = 16 * wave + lane / 4, lchunk = (lane % 4) ^ ((lane / 16) & 3);
    const int xoff = (m0 + lrow) * static_cast<int>(p.ld_x) + 16 * lchunk;
    const int woff = (n0 + lrow) * static_cast<int>(p.ld_w) + 16 * lchunk;
    const int xstride = 128 * static_cast<int>(p.ld_x), wstride = 128 * static_cast<int>(p.ld_w);
    // fragment reads: lane l of a 32-row block, substep st reads row l % 32, chunk 2 st + l / 32
    int rf[SUB];
#pragma unroll
    for (int st = 0; st < SUB; ++st) rf[st] = (lane % 32) * 64 + 16 * ((2 * st + lane / 32) ^ ((lane / 4) & 3));

    const auto issue = [&](int kt, unsigned char* xd, unsigned char* wd) {
#pragma unroll
        for (int i = 0; i < XLD; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (lds_void*)(xd + (wave + 8 * i) * 1024), 16, xoff, kt * KS + i * xstride, 0, 0);
#pragma unroll
        for (int i = 0; i < WLD; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wres, (lds_void*)(wd + (wave + 8 * i) * 1024), 16, woff, kt * KS + i * wstride, 0, 0);
    };
    const auto barrier = [&]() {
        asm volatile("" ::: "memory");
        wait_vm_lgkm0<XLD + WLD>();  // leaves this step's loads in flight, covers the next step's
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    const i32x16 zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    i32x16 tot[MB][2];
#pragma unroll
    for (int i = 0; i < MB; ++i) tot[i][0] = tot[i][1] = zero16;

    const auto step = [&](int kt, auto jt) {
        constexpr int j = decltype(jt)::value;
        issue(min(kt + 2, KT - 1), xstage(std::integral_constant<int, (j + 2) % 3>{}), wstage(std::integral_constant<int, (j + 2) % 3>{}));
        __builtin_amdgcn_sched_barrier(0);
        if (kt < KT) {
            const unsigned char* xs = xstage(std::integral_constant<int, j>{});
            const unsigned char* ws = wstage(std::integral_constant<int, j>{});
#pragma unroll
            for (int st = 0; st < SUB; ++st) {
                u32x4 a[MB], b[2];
#pragma unroll
                for (int i = 0; i < MB; ++i)
                    a[i] = *reinterpret_cast<const u32x4*>(xs + (wm * MB + i) * 2048 + rf[st]);
#pragma unroll
                for (int q = 0; q < 2; ++q) b[q] = *reinterpret_cast<const u32x4*>(ws + (2 * wn + q) * 2048 + rf[st]);
#pragma unroll
                for (int i = 0; i < MB; ++i)
#pragma unroll
                    for (int q = 0; q < 2; ++q) tot[i][q] = mfma_i8_32(a[i], b[q], tot[i][q]);
            }
        }
        barrier();
    };

    issue(0, xs0, ws0);
    issue(min(1, KT - 1), xs1, ws1);
    asm volatile("" ::: "memory");
    wait_vm_lgkm0<XLD + WLD>();  // step 0's loads
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    for (int kt = 0; kt < KT; kt += 3) {
        step(kt, std::integral_constant<int, 0>{});
        step(kt + 1, std::integral_constant<int, 1>{});
        step(kt + 2, std::integral_constant<int, 2>{});
    }
    wait_vm_lgkm0<0>();  // no direct load may still be writing LDS when the block ends

    // y = (float(S) * sx[t]) * sw[n], float32 or binary16 (round to nearest even)
    if (m0 + BM <= p.t && n0 + BN <= p.n) {
        // a whole tile: no bounds checks; wave-uniform row and column bases, 32-bit lane offsets
        constexpr unsigned ES = YT == SEPAL_HIP_F16 ? 2 : 4;
        const int wmu = __builtin_amdgcn_readfirstlane(wm), wnu = __builtin_amdgcn_readfirstlane(wn);
        const unsigned lrow = 4u * static_cast<unsigned>(lane / 32);
        const unsigned voff = (lrow * static_cast<unsigned>(p.ld_y) + lane % 32) * ES;
        const unsigned xoff = lrow * static_cast<unsigned>(p.ld_xs) * 4u;
        float sw[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) sw[q] = p.ws[static_cast<std::size_t>(n0 + 64 * wn + 32 * q + lane % 32) * p.ld_ws];
        char* const yb = static_cast<char*>(p.y);
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const std::size_t row = static_cast<std::size_t>(m0 + wmu * 32 * MB + i * 32 + 8 * (r / 4) + (r % 4));
                const float sx = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(p.xs + row * p.ld_xs) + xoff);
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const float v = __fmul_rn(__fmul_rn(static_cast<float>(tot[i][q][r]), sx), sw[q]);
                    char* const dst = yb + (row * p.ld_y + n0 + 64 * wnu + 32 * q) * ES + voff;
                    if constexpr (YT == SEPAL_HIP_F16) *reinterpret_cast<unsigned short*>(dst) = f32_to_f16_bits(v);
                    else *reinterpret_cast<float*>(dst) = v;
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + wm * 32 * MB + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
            if (row >= p.t) continue;
            const float sx = p.xs[static_cast<std::size_t>(row) * p.ld_xs];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int col = n0 + 64 * wn + 32 * q + lane % 32;
                if (col >= p.n) continue;
                const float v = __fmul_rn(__fmul_rn(static_cast<float>(tot[i][q][r]), sx), p.ws[static_cast<std::size_t>(col) * p.ld_ws]);
                const std::size_t idx = static_cast<std::size_t>(row) * p.ld_y + col;
                if constexpr (YT == SEPAL_HIP_F16) static_cast<unsigned short*>(p.y)[idx] = f32_to_f16_bits(v);
                else static_cast<float*>(p.y)[idx] = v;
            }
        }
}

// ---- launch ----------------------------------------------------------------------------------------------------------

inline Params make_params(const GemmArgs& a) {
    Params p{};
    p.x = reinterpret_cast<const signed char*>(a.x);
    p.ld_x = a.ld_x;
    p.xs = a.xs;
    p.ld_xs = a.ld_xs;
    int shift = 0;
    while ((static_cast<std::size_t>(128) << shift) < a.act_block) ++shift;
    p.act_shift = shift;
    p.w = reinterpret_cast<const signed char*>(a.w);
    p.ld_w = a.ld_w;
    p.ws = a.s;
    p.ld_ws = a.ld_s;
    p.y = a.y;
    p.ld_y = a.ld_y;
    p.t = static_cast<int>(a.t);
    p.n = static_cast<int>(a.n);
    p.k = static_cast<int>(a.k);
    p.sums = a.sums;
    p.ys = a.ys;
    p.ld_ys = a.ld_ys;
    return p;
}

// Compute units of the current device (cached per device).
inline int device_cus() {
    static std::atomic<int> cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) throw LaunchError("gemm_s8: hipGetDevice failed");
    if (dev < 64) {
        const int known = cached[dev].load(std::memory_order_relaxed);
        if (known > 0) return known;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        throw LaunchError("gemm_s8: device query failed");
    if (dev < 64) cached[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

template <int EP, int YT, bool PT, int MODE>
void launch_big(const GemmArgs& a, hipStream_t stream) {
    Params p = make_params(a);
    p.tiles_m = static_cast<int>((a.t + 127) / 128);
    p.tiles_n = static_cast<int>((a.n + 255) / 256);
    const std::size_t x_bytes = (a.t - 1) * a.ld_x + a.k, w_bytes = (a.n - 1) * a.ld_w + a.k;
    const std::size_t ws_bytes = MODE == MODE_CHAIN ? ((a.n - 1) * a.ld_s + a.k / 128) * 4 : 0;
    const std::size_t xs_bytes = MODE == MODE_CHAIN ? ((a.t - 1) * a.ld_xs + a.k / a.act_block) * 4 : 0;
    const std::size_t lim = std::size_t{1} << 31;
    if constexpr (MODE == MODE_CHAIN) {
        if (x_bytes < lim && w_bytes < lim && ws_bytes < lim && xs_bytes < lim) {
            const ChainParams cp{p, static_cast<unsigned>(x_bytes), static_cast<unsigned>(w_bytes),
                                 static_cast<unsigned>(ws_bytes), static_cast<unsigned>(xs_bytes)};
            // persistent: at most one block per CU, a whole number of blocks per XCD (the kernel's stride through its
            // XCD's tiles is grid / 8, so it must be at least 1; blocks whose range is empty leave at once)
            const int tiles = p.tiles_m * p.tiles_n;
            const int grid = 8 * std::max(1, std::min((tiles + 7) / 8, device_cus() / 8));
            if (grid % 8 != 0 || grid < 8) throw LaunchError("gemm_q8: persistent grid must be a positive multiple of 8");
            gemm_chain<EP, YT, PT><<<dim3(grid), dim3(512), 0, stream>>>(cp);
            check_launch("gemm_q8 large-M kernel launch");
            return;
        }
    }
    gemm_big<EP, YT, PT, MODE><<<dim3(p.tiles_m * p.tiles_n), dim3(512), 0, stream>>>(p);
    check_launch("gemm_q8 large-M kernel launch");
}

template <int EP, int YT, bool PT>
void dispatch_path(const GemmArgs& a, hipStream_t stream) {
    if constexpr (EP == SEPAL_HIP_SWIGLU && YT == SEPAL_HIP_F32) {
        // T <= 16 by default: the q8 stack's gate/up pass where it takes the shape
        SmallGemmPlan plan;
        if (a.config < 0 && a.t <= 16 && small_gemm_plan_q8(a, plan)) {
            launch_small_gemm_q8(a, plan, stream);
            return;
        }
    } else if constexpr (EP != SEPAL_HIP_SWIGLU) {
        // ... and its int8-X pass with K-parts for Store / Add
        SmallGemmPlan plan;
        if (a.config < 0 && a.t <= 16 && small_gemm_plan_q8_parts(a, plan)) {
            launch_small_gemm_q8_parts(a, plan, stream);
            return;
        }
    }
    const bool small = a.config == 1 || (a.config < 0 && q8_streams(a.t, a.n));
    if (small) launch_stream_q8(a, stream);
    else launch_big<EP, YT, PT, MODE_CHAIN>(a, stream);
}

template <bool PT>
void dispatch_ep(const GemmArgs& a, hipStream_t stream) {
    switch (a.epilogue) {
    case SEPAL_HIP_STORE: dispatch_path<SEPAL_HIP_STORE, SEPAL_HIP_F32, PT>(a, stream); break;
    case SEPAL_HIP_ADD: dispatch_path<SEPAL_HIP_ADD, SEPAL_HIP_F32, PT>(a, stream); break;
    default:
        switch (a.y_type) {
        case SEPAL_HIP_F32: dispatch_path<SEPAL_HIP_SWIGLU, SEPAL_HIP_F32, PT>(a, stream); break;
        case SEPAL_HIP_BF16: dispatch_path<SEPAL_HIP_SWIGLU, SEPAL_HIP_BF16, PT>(a, stream); break;
        default: dispatch_path<SEPAL_HIP_SWIGLU, SEPAL_HIP_F16, PT>(a, stream); break;
        }
    }
}

} // namespace q8

void launch_gemm_q8(const GemmArgs& a, hipStream_t stream) {
    if (a.act_block == a.k && a.k != 128) q8::dispatch_ep<true>(a, stream);
    else q8::dispatch_ep<false>(a, stream);
}

void launch_gemm_q8_swiglu_q8(const GemmArgs& a, hipStream_t stream) {
    if (a.act_block == a.k && a.k != 128) q8::launch_big<kSwigluQ8, SEPAL_HIP_F32, true, q8::MODE_CHAIN>(a, stream);
    else q8::launch_big<kSwigluQ8, SEPAL_HIP_F32, false, q8::MODE_CHAIN>(a, stream);
}

namespace q8 {


// 256 x 256 tiles when they fill the chip at least once, K is a multiple of 128 and every offset fits 32 bits; the last partial round, when
// more than a quarter full and small enough, as 128 x 256 halves in a second launch.
template <int YT>
bool launch_s8_big(const GemmArgs& a, hipStream_t stream) {
    const std::size_t tiles_m = (a.t + 255) / 256, tiles_n = (a.n + 255) / 256;
    const int cus = device_cus();
    if (tiles_m * tiles_n < static_cast<std::size_t>(cus) || a.k % 128 != 0) return false;
    if ((a.t + 256) * a.ld_x >= (std::size_t{1} << 31) || (a.n + 256) * a.ld_w >= (std::size_t{1} << 31)) return false;
    S8Params p{};
    p.x = static_cast<const signed char*>(a.x);
    p.ld_x = a.ld_x;
    p.xs = a.xs;
    p.ld_xs = a.ld_xs;
    p.w = reinterpret_cast<const signed char*>(a.w);
    p.ld_w = a.ld_w;
    p.ws = a.s;
    p.ld_ws = a.ld_s;
    p.y = a.y;
    p.ld_y = a.ld_y;
    p.t = static_cast<int>(a.t);
    p.n = static_cast<int>(a.n);
    p.k = static_cast<int>(a.k);
    p.tiles_m = static_cast<int>(tiles_m);
    p.tiles_n = static_cast<int>(tiles_n);
    p.x_bytes = (a.t - 1) * a.ld_x + a.k;
    p.w_bytes = (a.n - 1) * a.ld_w + a.k;
    const int total = p.tiles_m * p.tiles_n, full = total / cus * cus, rest = total - full;
    const bool split = rest > cus / 4 && full > 0 && 2 * rest <= cus;
    p.id0 = 0;
    p.count = split ? full : total;
    gemm_s8_big<YT, 4><<<dim3(p.count), dim3(512), 0, stream>>>(p);
    if (split) {
        S8Params q = p;
        q.id0 = full;
        q.count = rest;
        gemm_s8_big<YT, 2><<<dim3(2 * rest), dim3(512), 0, stream>>>(q);
    }
    check_launch("gemm_s8 large-M kernel launch");
    return true;
}

} // namespace q8

void launch_gemm_s8(const GemmArgs& a, hipStream_t stream) {
    if (a.y_type == SEPAL_HIP_F16) {
        if (!q8::launch_s8_big<SEPAL_HIP_F16>(a, stream)) q8::launch_big<SEPAL_HIP_STORE, SEPAL_HIP_F16, true, q8::MODE_WHOLE>(a, stream);
    } else {
        if (!q8::launch_s8_big<SEPAL_HIP_F32>(a, stream)) q8::launch_big<SEPAL_HIP_STORE, SEPAL_HIP_F32, true, q8::MODE_WHOLE>(a, stream);
    }
}

void launch_gemm_q8y(const GemmArgs& a, hipStream_t stream) {
    switch (a.epilogue) {
    case SEPAL_HIP_STORE: q8::launch_big<SEPAL_HIP_STORE, SEPAL_HIP_F32, true, q8::MODE_WHOLE_Y>(a, stream); break;
    case SEPAL_HIP_ADD: q8::launch_big<SEPAL_HIP_ADD, SEPAL_HIP_F32, true, q8::MODE_WHOLE_Y>(a, stream); break;
    default:
        switch (a.y_type) {
        case SEPAL_HIP_F32: q8::launch_big<SEPAL_HIP_SWIGLU, SEPAL_HIP_F32, true, q8::MODE_WHOLE_Y>(a, stream); break;
        case SEPAL_HIP_BF16: q8::launch_big<SEPAL_HIP_SWIGLU, SEPAL_HIP_BF16, true, q8::MODE_WHOLE_Y>(a, stream); break;
        default: q8::launch_big<SEPAL_HIP_SWIGLU, SEPAL_HIP_F16, true, q8::MODE_WHOLE_Y>(a, stream); break;
        }
    }
}

void launch_q8_group_sums(const GemmArgs& a, hipStream_t stream) {
    // at T <= 16 (config -1) the M <= 16 stack's pass kernels, whose int8 MFMAs the q8 stack and the single q8 calls at
    // those sizes run; else the large-M kernel body
    if (a.config < 0 && small_q8_group_sums(a, stream)) return;
    q8::launch_big<SEPAL_HIP_STORE, SEPAL_HIP_F32, true, q8::MODE_SUMS>(a, stream);
}

} // namespace sepal::hip
