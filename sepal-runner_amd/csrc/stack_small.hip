// The M <= 16 layer of the MLP stack (gpu-w8g, and its gpu-q8w form): three launches per layer, no cross-block
// hand-off inside a kernel. The same pass kernels also run single multiplies at T <= 16 (sepal_hip_gemm_w8g and
// sepal_hip_gemm_q8 at the default config, end of this file): SwiGLU straight to Y, Store / Add through K-parts and an
// in-order parts sum.
//
// At 16 tokens each layer is a single pass over 77 MB of int8 weights and scales, so the kernels are shaped to keep
// every CU streaming its share of weights for the whole kernel:
//   tiles  (gate/up, SwiGLU): one block of 16 waves per CU, and each block owns whole 16-row weight tiles (8 gate rows
//          and the 8 up rows of the same features) over the full K, 4 or 5 tiles per CU at the model's shape. 4 loader
//          waves stage the 16 X rows straight into LDS (their requests issued before any weight request) and the
//          block's scales, while the 12 worker waves already have every weight load of their pairs in flight and wait
//          for the loaders' flag; the block's (tile, group) pairs are split evenly
//          over the workers, and their partial tiles are added in LDS in worker order, then SwiGLU. Weight loads take
//          whole 128-byte lines (8 rows per instruction) and pass through a per-worker LDS transpose into the MFMA
//          layout.
//   parts  (down): the (K-part, column tile) units are dealt out evenly to the blocks, K-part major so that a
//          block's units share one slice of H; each unit's sum is written to a partial buffer P[part][row][col].
//   finish: one block per row adds the K-parts in order (y, float32), then runs the cpu-q8 RMSNorm on it with the
//          reference's summation order and writes the next layer's bf16 input (and, for q8, its int8 form).
// Per (tile or unit, group) pair the MFMA sum of the group (weights widened exactly to bf16 / binary16, float32
// accumulate) is scaled by the group's scale and added: y = sum_g s_g * P_g (proofs/GpuTrack/GpuTrack/GroupQuant.lean:
// 38-50), within float32 rounding of the reference's fmaf chain (runner/cuda/src/gemm_simt_kernels.cu:172-200).
// The q8 form multiplies int8 X (H quantized while the down pass stages it) by the int8 weights on int8 MFMAs: exact
// int32 group sums, then the cpu-q8 float chain per group.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "gemm_kernels.hpp"

namespace sepal::hip {
namespace stack {

constexpr int kWaves = 16, kThreads = 64 * kWaves;
constexpr int kLoaders = 4;                  // waves that stage X and the scales
constexpr int kWorkers = kWaves - kLoaders;  // waves that load weights and multiply
constexpr int kPairs = 9;   // (tile or unit, group) pairs one worker holds; all their loads are in flight at once
constexpr int kSlots = 3;   // tiles or units a worker's pairs may touch: 1 + ceil((kPairs - 1) / 4) with >= 4 groups per tile
constexpr int kScaleLoads = (kWorkers * kPairs * 16 + 64 * kLoaders - 1) / (64 * kLoaders);  // per loader thread

__device__ __forceinline__ f32x4 mfma16(int xt, const u32x4 a, const u32x4 b, f32x4 c) {
    if (xt == SEPAL_HIP_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void global_void;

// Activation type of the gpu-q8w stack: int8 X (and int8 H, quantized by the down pass's loaders) on int8 MFMAs.
constexpr int kActI8 = 8;
// The same with the multiply's X already int8 in every pass (one q8 Store / Add multiply: K-parts of int8 X).
constexpr int kActI8X = 9;

// The activation quantizer's rounding (rule RECIPROCAL: rint(v / scale) as v * (1 / scale), clamped to +-127), as
// quantize_rows applies it (runner/src/cpu/gemm.cpp pack_acts).
__device__ __forceinline__ int quantize_act(float v, float inverse) {
    float r = __builtin_rintf(__fmul_rn(v, inverse));
    r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
    return static_cast<int>(r);
}

struct PassParams {
    const unsigned short* x;  // [T, ld_x] bf16 / binary16; q8 gate/up: int8 [T, ld_x]
    std::size_t ld_x;
    const signed char* w;     // [N, ld_w]
    std::size_t ld_w;
    const float* s;           // [N, ld_s]
    std::size_t ld_s;
    void* y;                  // tiles: H [T, ld_y] of y_type; parts: P [parts][T][ld_y] float32
    std::size_t ld_y;
    int t, n, k;
    int tiles;                // weight tiles (16 rows each)
    int parts;                // K-parts (1 for the tiles pass)
    int per_block;            // tiles per block; a block's tiles share one K-part
    int blocks_per_part;      // ceil(tiles / per_block)
    // q8 only
    const float* xs;          // gate/up: X scales [T, ld_xs], one per token or per 128 columns
    std::size_t ld_xs;
    int per_token;            // 1: one activation scale per token; 0: one per 128 columns
    const float* xf;          // down: H float32 [T, ld_x], quantized here (per 128 columns)
    int h16;                  // the stack's per-token form: the gate/up pass writes H in binary16 (its row maxima over
                              // the rounded values), and the down pass stages binary16 H from x
    const float* hmax;        // down, per token: the gate/up pass's partial row maxima of |H| [T, hmax_blocks]
    int hmax_blocks;
    float* pmax;              // gate/up, per token: this pass's partial row maxima [T, gridDim.x]
    std::int32_t* sums;       // q8, when set: only the exact int32 group sums, sums[g][T][N] (no chain, no epilogue)
};

// Weight row of column c (0..15) of a tile. SwiGLU tiles take 8 gate rows and the 8 up rows of the same features in the
// 64-row gate/up interleave (packed row 128 b + r is gate feature 64 b + r, row 128 b + 64 + r is up feature 64 b + r).
template <bool SWIGLU>
__device__ __forceinline__ int tile_row(int tile, int c) {
    if constexpr (SWIGLU) {
        const int b = tile / 8, r0 = 8 * (tile % 8);
        return c < 8 ? 128 * b + r0 + c : 128 * b + 64 + r0 + (c - 8);
    } else {
        return 16 * tile + c;
    }
}

constexpr int kXChunks = 6;  // 16-byte X chunks per lane of a staged row: 64 x 6 x 8 = 3072 columns at most

// The stack's per-token form (h16): binary16 H and one scale per row (the maximum of the gate/up pass's partial
// maxima), so no group maxima. A row's loads: 8 values a lane per 16-byte load, 16 lanes per 128 columns (NQ loads
// cover 4 NQ groups), and its partial maxima; staging widens and quantizes it into LDS.
template <int NQ>
struct H16Row {
    uint4 hb[NQ];
    float pm[4];  // 64 lanes x 4: the gate/up grid has at most 256 blocks
};

template <int NQ>
__device__ __forceinline__ void h16_issue(const PassParams& p, int g_lo, int gpt, int r, int lane, H16Row<NQ>& h) {
    const int rs = min(r, p.t - 1);
    const unsigned short* hrow = p.x + static_cast<std::size_t>(rs) * p.ld_x + 128 * g_lo;
#pragma unroll
    for (int e = 0; e < NQ; ++e)
        h.hb[e] = *reinterpret_cast<const uint4*>(hrow + 128 * min(4 * e + lane / 16, gpt - 1) + 8 * (lane % 16));
#pragma unroll
    for (int i = 0; i < 4; ++i)
        h.pm[i] = p.hmax[static_cast<std::size_t>(rs) * p.hmax_blocks + min(lane + 64 * i, p.hmax_blocks - 1)];
}

template <int NQ>
__device__ __forceinline__ void h16_stage(unsigned char* lds, float* xsc, int xpitch, int gpt, int r, int lane, const H16Row<NQ>& h) {
    float m = fmaxf(fmaxf(h.pm[0], h.pm[1]), fmaxf(h.pm[2], h.pm[3]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    const float rscale = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
    const float rinv = __fdiv_rn(1.0f, rscale);
    if (lane == 0) xsc[r] = rscale;
#pragma unroll
    for (int e = 0; e < NQ; ++e) {
        if (4 * e >= gpt) break;  // uniform
        const int g = 4 * e + lane / 16;
        const unsigned w[4] = {h.hb[e].x, h.hb[e].y, h.hb[e].z, h.hb[e].w};
        unsigned packed[2] = {0u, 0u};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float v = f16_bits_to_f32(static_cast<unsigned short>((w[j / 2] >> (16 * (j % 2))) & 0xFFFFu));
            packed[j / 4] |= (static_cast<unsigned>(quantize_act(v, rinv)) & 0xFFu) << (8 * (j % 4));
        }
        if (g < gpt) *reinterpret_cast<uint2*>(lds + r * xpitch + 128 * g + 8 * (lane % 16)) = make_uint2(packed[0], packed[1]);
    }
}

// The q8 down pass's staging of H rows 4 w .. 4 w + 3 (w = loader wave), ROWS rows per round trip: NQ float4 loads
// per lane and row cover 2 NQ blocks of 128 columns (NQ = ceil(gpt / 2) rounded up to an instantiated size).
template <int NQ, int ROWS>
__device__ __forceinline__ void stage_h_q8(const PassParams& p, unsigned char* lds, float* xsc, int xpitch, int g_lo, int gpt,
                                           int row0, int nrows, int lane) {
    constexpr int kMaxPartials = 4;  // 64 lanes x 4: the gate/up grid has at most 256 blocks
#pragma unroll 1
    for (int rr = 0; rr < nrows; rr += ROWS) {
        float4 hv[ROWS][NQ];
        float pm[ROWS][kMaxPartials];
#pragma unroll
        for (int h = 0; h < ROWS; ++h) {
            const int rs = min(row0 + rr + h, p.t - 1);
            const float* hrow = p.xf + static_cast<std::size_t>(rs) * p.ld_x + 128 * g_lo;
#pragma unroll
            for (int e = 0; e < NQ; ++e)
                hv[h][e] = *reinterpret_cast<const float4*>(hrow + 128 * min(2 * e + lane / 32, gpt - 1) + 4 * (lane % 32));
            if (p.per_token) {
#pragma unroll
                for (int i = 0; i < kMaxPartials; ++i)
                    pm[h][i] = p.hmax[static_cast<std::size_t>(rs) * p.hmax_blocks + min(lane + 64 * i, p.hmax_blocks - 1)];
            }
        }
#pragma unroll
        for (int h = 0; h < ROWS; ++h) {
            const int r = row0 + rr + h;
            float rscale = 1.0f, rinv = 1.0f;
            if (p.per_token) {
                float m = fmaxf(fmaxf(pm[h][0], pm[h][1]), fmaxf(pm[h][2], pm[h][3]));
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
                rscale = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
                rinv = __fdiv_rn(1.0f, rscale);
                if (lane == 0) xsc[r] = rscale;
            }
#pragma unroll
            for (int e = 0; e < NQ; ++e) {
                if (2 * e >= gpt) break;  // uniform
                const int g = 2 * e + lane / 32;
                const float v[4] = {hv[h][e].x, hv[h][e].y, hv[h][e].z, hv[h][e].w};
                float scale = rscale, inv = rinv;
                if (!p.per_token) {
                    float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
                    for (int o = 16; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 32));
                    scale = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
                    inv = __fdiv_rn(1.0f, scale);
                }
                unsigned packed = 0u;
#pragma unroll
                for (int j = 0; j < 4; ++j) packed |= (static_cast<unsigned>(quantize_act(v[j], inv)) & 0xFFu) << (8 * j);
                if (g < gpt) {
                    *reinterpret_cast<unsigned*>(lds + r * xpitch + 128 * g + 4 * (lane % 32)) = packed;
                    if (!p.per_token && lane % 32 == 0) xsc[r * gpt + g] = scale;
                }
            }
        }
    }
}

// One multiply pass over a block of weight tiles and one K-part (the gate/up pass: SWIGLU, one part covering K, the
// output H; the down pass: several parts, the output P[part]). XT is the activation type, YT the SwiGLU output type.
//
// Every wave stages one X row (one block barrier, before any weight load). Then waves 0 .. kLoaders - 1 stage the
// block's scales in LDS and raise an LDS flag; waves kLoaders .. 15 (the workers) issue every weight load of their
// pairs at once, wait for the flag, and multiply. The weights are in flight while the scales arrive, and no worker's
// load issue (which stalls when the memory queues are full) holds up a barrier.
// STREAM: the weights in the stream layout (make_stream_layout): each (tile, group) pair's 2 KB contiguous, already in
// the MFMA operand order, so a pair is two 1 KB loads and needs no LDS transpose. H16: the q8 down pass of the stack's
// per-token form (binary16 H, p.h16 set), an instance of its own so that the per-128 form keeps its own code.
template <int XT, bool SWIGLU, int YT, bool STREAM = false, bool H16 = false>
__global__ void __launch_bounds__(kThreads) pass_kernel(const PassParams p) {
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ unsigned ready;
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int groups = p.k / 128;
    const int part = blockIdx.x / p.blocks_per_part;
    const int tile0 = (blockIdx.x % p.blocks_per_part) * p.per_block;
    const int ntiles = min(p.per_block, p.tiles - tile0);
    const int g_lo = part * groups / p.parts, g_hi = (part + 1) * groups / p.parts;
    const int gpt = g_hi - g_lo;              // groups per tile in this part
    const int kw = 128 * gpt;                 // staged X columns [128 g_lo, 128 g_hi)
    constexpr bool Q8 = XT == kActI8 || XT == kActI8X;
    const int xpitch = (Q8 ? kw : 2 * kw) + 16;  // bytes per staged row (padded: an operand read's 16 rows hit distinct banks)
    float* red = reinterpret_cast<float*>(lds + 16 * xpitch);  // [kWorkers][kSlots][16 x 16]
    float* scl = red + kWorkers * kSlots * 256;                 // [block tile][16 rows][gpt] scales
    unsigned char* tbuf = reinterpret_cast<unsigned char*>(scl + kWorkers * kPairs * 16);  // [worker][2 KB] transposes
    float* xsc = reinterpret_cast<float*>(tbuf + kWorkers * 2048);  // q8: activation scales [16 rows][gpt] (per token [16])
    // the block's (tile, group) pairs, tile major, dealt to the workers in runs of `per` (the last may get none)
    const int total = ntiles * gpt;
    const int per = (total + kWorkers - 1) / kWorkers;
    __shared__ unsigned row_max[16];  // q8 gate/up, per token: |H| maxima of this block's outputs (float bits)
    if (tid == 0) ready = 0u;
    if (tid < 16) row_max[tid] = 0u;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the counter is zero before the barrier below lets any wave count
    // ---- X. The loader waves stage the rows straight from global memory into LDS (direct loads, no registers; 4 rows
    // a wave), and their requests are issued before any weight request of the block (a bare barrier orders the issue,
    // not the arrival): behind a weight burst these loads would wait in the memory queues, and waiting for them before
    // the burst (as a block barrier would) leaves the weight stream idle for their round trip. The workers wait for
    // the loaders' flag. Rows past T are not loaded (each MFMA output row depends on its own X row only, and those
    // rows feed only outputs that are never stored). The q8 down pass quantizes H while it stages it: per 128 columns
    // every wave one row, ahead of the burst; in the stack's per-token form (binary16 H, K-parts of up to 16 groups)
    // the loader waves issue their 4 rows' loads before any weight request, as for X, and quantize the rows while the
    // weights stream (all 16 rows: guarding them measured slower). ----
    constexpr bool kQ8Down = XT == kActI8 && !SWIGLU;
    [[maybe_unused]] H16Row<4> hrows[4];
    const bool h16_loaders = kQ8Down && H16 && gpt <= 16;  // (uniform)
    constexpr bool kEarly = !(XT == kActI8 && !SWIGLU);  // X loads in flight under the weight issue
    float xsv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // the loaders' share of the block's weight scales (row runs of gpt words)
    float sv[kScaleLoads];
    const auto load_scales = [&] {
#pragma unroll
        for (int e = 0; e < kScaleLoads; ++e) {
            const int idx = min(tid + e * 64 * kLoaders, total * 16 - 1);
            const int tl = idx / (16 * gpt), rem = idx % (16 * gpt);
            const int row = min(tile_row<SWIGLU>(tile0 + tl, rem / gpt), p.n - 1);
            sv[e] = p.s[static_cast<std::size_t>(row) * p.ld_s + g_lo + rem % gpt];
        }
    };
    if constexpr (XT == kActI8 && !SWIGLU) {
        // q8 down: H (float32 per 128 columns; binary16 in the stack's per-token form) quantized as the activation
        // quantizer does (rule RECIPROCAL, scale = max / 127), per 128 columns or with the row maximum of the gate/up
        // pass's partial maxima (per token)
        if (h16_loaders) {
            if (wave < kLoaders) {
#pragma unroll
                for (int j = 0; j < 4; ++j) h16_issue<4>(p, g_lo, gpt, 4 * wave + j, lane, hrows[j]);
            }
            __builtin_amdgcn_s_barrier();  // the loaders' H requests are issued before any weight request
        } else if (H16) {
            if (wave < p.t) {
                H16Row<6> h6;
                h16_issue<6>(p, g_lo, gpt, wave, lane, h6);
                h16_stage<6>(lds, xsc, xpitch, gpt, wave, lane, h6);
            }
            __syncthreads();
        } else {
            if (wave < p.t) {
                if (gpt <= 14) stage_h_q8<7, 1>(p, lds, xsc, xpitch, g_lo, gpt, wave, 1, lane);
                else stage_h_q8<12, 1>(p, lds, xsc, xpitch, g_lo, gpt, wave, 1, lane);
            }
            __syncthreads();
        }
    } else {
        if (wave < kLoaders) {
            const int chunks = Q8 ? kw / 16 : kw / 8;  // 16-byte chunks of a row
            const int esz = Q8 ? 1 : 2;
            const auto stage_rows = [&](auto all_live) __attribute__((always_inline)) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r = 4 * wave + j, xr = min(r, p.t - 1);
                    const unsigned char* xrow = reinterpret_cast<const unsigned char*>(p.x) + (static_cast<std::size_t>(xr) * p.ld_x + 128 * g_lo) * esz;
#pragma unroll
                    for (int e = 0; e < (Q8 ? kXChunks / 2 : kXChunks); ++e)
                        if ((decltype(all_live)::value || r < p.t) && lane + 64 * e < chunks)
                            __builtin_amdgcn_global_load_lds((global_void*)(xrow + 16 * (lane + 64 * e)),
                                                             (lds_void*)(lds + r * xpitch + 1024 * e), 16, 0, 0);
                    if constexpr (Q8) {
                        const int nsc = p.per_token ? 1 : gpt;
                        xsv[j] = p.xs[static_cast<std::size_t>(xr) * p.ld_xs + (p.per_token ? 0 : g_lo + min(lane, nsc - 1))];
                    }
                }
            };
            // (a wave whose four rows are all below T runs the unguarded loop)
            if (4 * wave + 3 < p.t) stage_rows(std::true_type{});
            else stage_rows(std::false_type{});
        }
        __builtin_amdgcn_s_barrier();  // the loaders' X requests are issued before any weight request
    }

    if (wave < kLoaders) {
        // ---- loaders: the block's weight scales into LDS (issued beside the workers' weights: ahead of them they
        // measured slower), then X (the q8 activation scales too) has landed ----
        load_scales();
#pragma unroll
        for (int e = 0; e < kScaleLoads; ++e)
            if (tid + e * 64 * kLoaders < total * 16) scl[tid + e * 64 * kLoaders] = sv[e];
        if constexpr (kEarly) {
            if constexpr (Q8) {
                const int nsc = p.per_token ? 1 : gpt;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (lane < nsc) xsc[p.per_token ? 4 * wave + j : (4 * wave + j) * gpt + lane] = xsv[j];
            }
            __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) lgkmcnt(0): the direct X loads have landed in LDS
        }
        if constexpr (kQ8Down) {
            if (h16_loaders) {
#pragma unroll
                for (int j = 0; j < 4; ++j) h16_stage<4>(lds, xsc, xpitch, gpt, 4 * wave + j, lane, hrows[j]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
        if (lane == 0) __hip_atomic_fetch_add(&ready, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    } else {
        const int wk = wave - kLoaders;
        const int q0 = min(wk * per, total), q1 = min(q0 + per, total);
        const int n_pairs = q1 - q0;
        const int first_tile = min(q0, total - 1) / gpt;  // block-local
        // ---- every weight load of this worker's pairs at once (clamped, unconditional). The pairs touch at most
        // kSlots consecutive tiles; their row pointers are formed once, and the (tile, group) walk is wave-uniform;
        // past the worker's share it stays on its last pair (the same addresses again, never multiplied). ----
        // A pair's weights are 16 rows x 128 bytes, loaded as two instructions of 8 rows x 128 bytes (whole cache
        // lines: lane l takes row l / 8 and 16-byte chunk l % 8); the second 8 rows are kRowStep rows past the first.
        constexpr int kRowStep = SWIGLU ? 64 : 8;
        const signed char* wrow[kSlots];
#pragma unroll
        for (int j = 0; j < kSlots; ++j) {
            const int tile = tile0 + min(first_tile + j, ntiles - 1);
            const std::size_t row = static_cast<std::size_t>(tile_row<SWIGLU>(tile, lane / 8));  // the plan keeps rows < N
            wrow[j] = p.w + row * p.ld_w + 16 * (lane % 8);
        }
        u32x4 wb[kPairs][2];
        int pslot[kPairs], pg[kPairs];
        {
            const int qs = min(q0, total - 1);
            int slot = qs / gpt - first_tile, g = g_lo + qs % gpt;
#pragma unroll
            for (int i = 0; i < kPairs; ++i) {
                pslot[i] = slot;
                pg[i] = g;
                if (q0 + i + 1 < q1) {
                    if (++g == g_hi) {
                        g = g_lo;
                        ++slot;
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < kPairs; ++i) {
            if constexpr (STREAM) {
                // pair (tile, group): 2 KB at (tile * groups + group) * 2048, half h at + 1024 h, lane l's 16 bytes at
                // + 16 l: weight row tile_row(tile, l % 16), k = 128 group + 64 h + 16 (l / 16) .. + 15
                const std::size_t blk = static_cast<std::size_t>(tile0 + first_tile + pslot[i]) * groups + pg[i];
                const signed char* src = p.w + blk * 2048 + 16 * lane;
                wb[i][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
                wb[i][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 1024));
            } else {
                const signed char* src = wrow[0] + 128 * pg[i];
#pragma unroll
                for (int j = 1; j < kSlots; ++j)
                    if (pslot[i] == j) src = wrow[j] + 128 * pg[i];
                wb[i][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
                wb[i][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + kRowStep * p.ld_w));
            }
        }
        // ---- X and the scales are staged ----
        while (__hip_atomic_load(&ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < static_cast<unsigned>(kLoaders))
            __builtin_amdgcn_s_sleep(1);

        // ---- multiply: per pair, the weights pass through this worker's 2 KB of LDS into the MFMA layout (row r's
        // chunk c at r * 128 + ((c + r / 2) % 8) * 16: the writes and the reads hit 16 bank groups per 16 lanes), then
        // four MFMAs over the group's 128 k (lane quarter q holds k 16 q .. 16 q + 15 of each 64-k half: the same
        // permutation on both operands), then cur += s * P; the worker's pairs run tile by tile, and each finished tile
        // goes to its LDS slot [worker][slot][row][col] ----
        unsigned char* tb = tbuf + wk * 2048;
        const int wr_lo = (lane / 8) * 128 + ((lane % 8 + lane / 16) % 8) * 16;  // rows 0..7 (r / 2 = lane / 16)
        const int wr_hi = (8 + lane / 8) * 128 + ((lane % 8 + 4 + lane / 16) % 8) * 16;  // rows 8..15
        f32x4 cur = {0.0f, 0.0f, 0.0f, 0.0f};
        int cur_slot = 0;
        const auto flush = [&](int slot_) {
#pragma unroll
            for (int r = 0; r < 4; ++r) red[(wk * kSlots + slot_) * 256 + (4 * (lane / 16) + r) * 16 + lane % 16] = cur[r];
        };
#pragma unroll
        for (int i = 0; i < kPairs; ++i) {
            if (i >= n_pairs) continue;
            // (the walk above: pair i is group pg[i] of tile slot pslot[i]; a new tile starts where it wrapped to g_lo)
            const int gq = pg[i] - g_lo;  // = (q0 + i) mod gpt, without a division per pair
            if (i > 0 && gq == 0) {  // a new tile (wave-uniform)
                flush(cur_slot);
                ++cur_slot;
                cur = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
            const float sc = scl[((first_tile + pslot[i]) * 16 + lane % 16) * gpt + (pg[i] - g_lo)];
            const int kofs = 128 * gq;
            f32x4 prt = {0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (!STREAM) {
                *reinterpret_cast<u32x4*>(tb + wr_lo) = wb[i][0];
                *reinterpret_cast<u32x4*>(tb + wr_hi) = wb[i][1];
            }
            // the MFMA operand of half h: lane l's 16 bytes of weight row l % 16, k = 64 h + 16 (l / 16) .. + 15
            const auto wop = [&](int h) __attribute__((always_inline)) -> u32x4 {
                if constexpr (STREAM) return wb[i][h];
                const int rr = lane % 16, cc = 4 * h + lane / 16;
                return *reinterpret_cast<const u32x4*>(tb + rr * 128 + ((cc + rr / 2) % 8) * 16);
            };
            if constexpr (Q8) {
                // the int8 weights go to the MFMA as they are: the exact int32 group sum, then the cpu-q8 float chain
                // (runner/src/cpu/gemm_kernels_avx512.cpp:67-115): t = fma(f_g, ws_g, t) with one scale per token
                // (applied after the sum), fma(f_g, ws_g * xs_g, t) with one per 128 columns
                i32x4 acc = {0, 0, 0, 0};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const u32x4 wv = wop(h);
                    const u32x4 a = *reinterpret_cast<const u32x4*>(lds + (lane % 16) * xpitch + kofs + 64 * h + 16 * (lane / 16));
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, wv), acc, 0, 0, 0);
                }
                if (p.sums != nullptr) {
                    // the pair's group sums as they are: lane l holds token rows 4 (l / 16) + r of weight row
                    // (tile column) l % 16
                    const int wrow_n = tile_row<SWIGLU>(tile0 + first_tile + pslot[i], lane % 16);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int row = 4 * (lane / 16) + r;
                        if (row < p.t && wrow_n < p.n)
                            p.sums[(static_cast<std::size_t>(pg[i]) * p.t + row) * p.n + wrow_n] = acc[r];
                    }
                    continue;
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float s_r = p.per_token ? sc : __fmul_rn(sc, xsc[(4 * (lane / 16) + r) * gpt + gq]);
                    cur[r] = __builtin_fmaf(static_cast<float>(acc[r]), s_r, cur[r]);
                }
                continue;
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const u32x4 wv = wop(h);
                unsigned o[8];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    if constexpr (XT == SEPAL_HIP_BF16) s8x4_to_bf16x4(wv[c], o[2 * c], o[2 * c + 1]);
                    else s8x4_to_f16x4(wv[c], o[2 * c], o[2 * c + 1]);
                }
                const unsigned char* xr = lds + (lane % 16) * xpitch + 2 * (kofs + 64 * h + 16 * (lane / 16));
                const u32x4 a0 = *reinterpret_cast<const u32x4*>(xr);
                const u32x4 a1 = *reinterpret_cast<const u32x4*>(xr + 16);
                prt = mfma16(XT, a0, u32x4{o[0], o[1], o[2], o[3]}, prt);
                prt = mfma16(XT, a1, u32x4{o[4], o[5], o[6], o[7]}, prt);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) cur[r] = __builtin_fmaf(prt[r], sc, cur[r]);
        }
        if (n_pairs > 0) flush(cur_slot);
    }

    if (p.sums != nullptr) return;  // (uniform) the group sums are written
    // ---- per block-local tile: the workers that cover it, q / per over the tile's pairs; per worker: its first tile ----
    __shared__ int cover_lo[kWaves], cover_hi[kWaves], worker_first[kWorkers];
    if (tid < ntiles) {
        cover_lo[tid] = tid * gpt / per;
        cover_hi[tid] = ((tid + 1) * gpt - 1) / per;
    }
    if (tid < kWorkers) worker_first[tid] = min(tid * per, total - 1) / gpt;
    __syncthreads();
    // the tile's sum in worker order; tile tl sits in slot tl - (first tile of w) of worker w, which is slot 0 for every
    // worker after the first (it starts inside the tile)
    const auto sum_tile = [&](int tl, int e) {
        const int lo = cover_lo[tl], hi = cover_hi[tl];
        float v = red[(lo * kSlots + (tl - worker_first[lo])) * 256 + e];
#pragma unroll 4
        for (int w = lo + 1; w <= hi; ++w) v = __fadd_rn(v, red[w * kSlots * 256 + e]);
        return v;
    };
    if constexpr (Q8 && SWIGLU) {
        // H = SwiGLU(gate, up) in float32 (the gpu-q8w epilogue; binary16 when h16 is set), and, per token, this
        // block's row maxima of |H|
        float* hy = static_cast<float*>(p.y);
        for (int id = tid; id < ntiles * 16 * 8; id += kThreads) {
            const int tl = id / 128, r = (id / 8) % 16, i = id % 8;
            const int tile = tile0 + tl;
            const int f = 64 * (tile / 8) + 8 * (tile % 8) + i;
            if (r >= p.t || 2 * f >= p.n) continue;
            float g = sum_tile(tl, r * 16 + i), u = sum_tile(tl, r * 16 + 8 + i);
            if (p.per_token) {
                g = __fmul_rn(g, xsc[r]);
                u = __fmul_rn(u, xsc[r]);
            }
            // (per token, a form with no reference bits, the fast silu, as the large-M q8 kernels use it)
            const float hv = p.per_token ? swiglu_fast(g, u) : swiglu_cephes(g, u);
            if (p.h16) {
                // binary16 H, as the large-M per-token stack writes it; the maxima are over the rounded values
                const unsigned short hb = f32_to_f16_bits(hv);
                static_cast<unsigned short*>(p.y)[static_cast<std::size_t>(r) * p.ld_y + f] = hb;
                atomicMax(&row_max[r], __float_as_uint(fabsf(f16_bits_to_f32(hb))));
            } else {
                hy[static_cast<std::size_t>(r) * p.ld_y + f] = hv;
                if (p.per_token) atomicMax(&row_max[r], __float_as_uint(fabsf(hv)));
            }
        }
        if (p.per_token) {
            __syncthreads();
            if (tid < p.t) p.pmax[static_cast<std::size_t>(tid) * gridDim.x + blockIdx.x] = __uint_as_float(row_max[tid]);
        }
    } else if constexpr (Q8) {
        float* y = static_cast<float*>(p.y);
        for (int id = tid; id < ntiles * 256; id += kThreads) {
            const int tl = id / 256, r = (id / 16) % 16, c = id % 16;
            const int col = 16 * (tile0 + tl) + c;
            if (r >= p.t || col >= p.n) continue;
            const float v = sum_tile(tl, r * 16 + c);
            y[(static_cast<std::size_t>(part) * p.t + r) * p.ld_y + col] = p.per_token ? __fmul_rn(v, xsc[r]) : v;
        }
    } else if constexpr (SWIGLU) {
        // output (tile, row, feature i < 8) = swiglu(col i, col 8 + i)
        for (int id = tid; id < ntiles * 16 * 8; id += kThreads) {
            const int tl = id / 128, r = (id / 8) % 16, i = id % 8;
            const int tile = tile0 + tl;
            const int f = 64 * (tile / 8) + 8 * (tile % 8) + i;
            if (r >= p.t || 2 * f >= p.n) continue;
            const float g = sum_tile(tl, r * 16 + i), u = sum_tile(tl, r * 16 + 8 + i);
            store_out<YT>(p.y, static_cast<std::size_t>(r) * p.ld_y + f, swiglu_fast(g, u));
        }
    } else {
        float* y = static_cast<float*>(p.y);
        for (int id = tid; id < ntiles * 256; id += kThreads) {
            const int tl = id / 256, r = (id / 16) % 16, c = id % 16;
            const int col = 16 * (tile0 + tl) + c;
            if (r >= p.t || col >= p.n) continue;
            y[(static_cast<std::size_t>(part) * p.t + r) * p.ld_y + col] = sum_tile(tl, r * 16 + c);
        }
    }
}

// The stream layout of an int8 [n, k] weight matrix for the M <= 16 passes (n a multiple of 16, k of 128): pair (tile,
// group) is 2 KB at (tile * (k / 128) + group) * 2048; its half h, at + 1024 h, holds for lane l the 16 bytes of weight
// row tile_row(tile, l % 16) at k = 128 group + 64 h + 16 (l / 16) .. + 15 (the MFMA operand the pass kernels form
// through their LDS transpose). interleave: gate/up tiles of 8 gate and the 8 up rows of the same features. One thread
// moves one 16-byte item.
__global__ void __launch_bounds__(256) stream_layout_kernel(const signed char* __restrict__ w, std::size_t ld_w, int n, int k,
                                                            int interleave, signed char* __restrict__ out) {
    const std::size_t id = static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x;
    const int groups = k / 128;
    const std::size_t items = static_cast<std::size_t>(n / 16) * groups * 128;
    if (id >= items) return;
    const int l = static_cast<int>(id % 64), h = static_cast<int>((id / 64) % 2);
    const std::size_t blk = id / 128;
    const int g = static_cast<int>(blk % groups), tile = static_cast<int>(blk / groups);
    const int row = interleave ? tile_row<true>(tile, l % 16) : tile_row<false>(tile, l % 16);
    const u32x4 v = *reinterpret_cast<const u32x4*>(w + static_cast<std::size_t>(row) * ld_w + 128 * g + 64 * h + 16 * (l / 16));
    *reinterpret_cast<u32x4*>(out + id * 16) = v;
}

// y[r][c] = sum over the P parts (in order) of P[part][r][c]; then, if xn is set, xn[r] = bf16(RMSNorm(y[r])) with the
// cpu-q8 summation order (runner/src/cpu/elementwise.cpp:22-59) and eps. One block of 1024 threads per row; each
// thread's P partial loads are all in flight at once (P is a template argument, so no load repeats a part).
constexpr int kFinishParts = 16;

// With q set (the gpu-q8w stack), the bf16 values are also quantized as quantize_rows does (rule RECIPROCAL), with
// one scale per row (qblock = n) or per 128 columns (qblock = 128), into q [t, n] and qs [t, n / qblock].
template <int P>
__global__ void __launch_bounds__(1024) finish_kernel(const float* __restrict__ part, int t, int n, float* __restrict__ y,
                                                      std::uint16_t* __restrict__ xn, double eps, std::int8_t* __restrict__ q,
                                                      float* __restrict__ qs, int qblock) {
    extern __shared__ __align__(16) float row_buf[];  // [n]
    const int r = blockIdx.x, tid = threadIdx.x;
    for (int c4 = tid; c4 < n / 4; c4 += 1024) {
        float4 v[P];
#pragma unroll
        for (int q = 0; q < P; ++q)
            v[q] = *reinterpret_cast<const float4*>(part + (static_cast<std::size_t>(q) * t + r) * n + 4 * c4);
        float4 a = v[0];
#pragma unroll
        for (int q = 1; q < P; ++q) {
            a.x = __fadd_rn(a.x, v[q].x);
            a.y = __fadd_rn(a.y, v[q].y);
            a.z = __fadd_rn(a.z, v[q].z);
            a.w = __fadd_rn(a.w, v[q].w);
        }
        *reinterpret_cast<float4*>(row_buf + 4 * c4) = a;
        *reinterpret_cast<float4*>(y + static_cast<std::size_t>(r) * n + 4 * c4) = a;
    }
    if (xn == nullptr && q == nullptr) return;  // uniform over the block
    __syncthreads();
    // lanes 0..31 of wave 0 are the reference's 4 x 8 accumulator lanes: lane L adds c = L, L + 32, ..., then the
    // 8-wide tail on lanes 0..7
    __shared__ float inv_s;
    if (tid < 64) {
        const int L = tid % 32;
        float a = 0.0f;
        const int full = n / 32 * 32;
        if (tid < 32) {
            // forty reads in flight, then their forty links of the chain, in order (one LDS round trip per 1280
            // columns instead of one per 256)
            int c = 0;
            for (; c + 1280 <= full; c += 1280) {
                float v[40];
#pragma unroll
                for (int u = 0; u < 40; ++u) v[u] = row_buf[c + 32 * u + L];
#pragma unroll
                for (int u = 0; u < 40; ++u) a = __builtin_fmaf(v[u], v[u], a);
            }
            for (; c + 256 <= full; c += 256) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = row_buf[c + 32 * u + L];
#pragma unroll
                for (int u = 0; u < 8; ++u) a = __builtin_fmaf(v[u], v[u], a);
            }
            for (; c < full; c += 32) a = __builtin_fmaf(row_buf[c + L], row_buf[c + L], a);
            for (c = full; c + 8 <= n; c += 8)
                if (L < 8) a = __builtin_fmaf(row_buf[c + L], row_buf[c + L], a);
        }
        const int l8 = L % 8;
        const float a0 = __shfl(a, l8), a1 = __shfl(a, 8 + l8), a2 = __shfl(a, 16 + l8), a3 = __shfl(a, 24 + l8);
        const float sl = __fadd_rn(__fadd_rn(a0, a1), __fadd_rn(a2, a3));
        const float sl4 = __shfl(sl, (l8 + 4) % 8);
        const float h = __fadd_rn(sl, sl4);
        const float h0 = __shfl(h, 0), h1 = __shfl(h, 1), h2 = __shfl(h, 2), h3 = __shfl(h, 3);
        const float sum = __fadd_rn(__fadd_rn(h0, h2), __fadd_rn(h1, h3));
        if (tid == 0) {
            const double mean = static_cast<double>(sum) / static_cast<double>(n);
            inv_s = static_cast<float>(1.0 / __builtin_sqrt(mean + eps));
        }
    }
    __syncthreads();
    const float inv = inv_s;
    if (xn != nullptr)
        for (int c = tid; c < n; c += 1024) xn[static_cast<std::size_t>(r) * n + c] = f32_to_bf16_bits(__fmul_rn(row_buf[c], inv));
    if (q == nullptr) return;
    // the bf16-rounded values, their maxima (per row, or per 128 columns: two waves per block of 128), the int8 values
    __shared__ float wmax[16];
    __shared__ float rmax_s;
    const int wave = tid / 64, lane = tid % 64;
    if (qblock != 128) {
        float m = 0.0f;
        for (int c = tid; c < n; c += 1024) m = fmaxf(m, fabsf(bf16_bits_to_f32(f32_to_bf16_bits(__fmul_rn(row_buf[c], inv)))));
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        if (lane == 0) wmax[wave] = m;
        __syncthreads();
        if (tid == 0) {
            float a = wmax[0];
            for (int w = 1; w < 16; ++w) a = fmaxf(a, wmax[w]);
            rmax_s = a;
        }
        __syncthreads();
        const float scale = rmax_s > 0.0f ? __fdiv_rn(rmax_s, 127.0f) : 1.0f;
        const float inverse = __fdiv_rn(1.0f, scale);
        if (tid == 0) qs[r] = scale;
        for (int c = tid; c < n; c += 1024)
            q[static_cast<std::size_t>(r) * n + c] =
                static_cast<std::int8_t>(quantize_act(bf16_bits_to_f32(f32_to_bf16_bits(__fmul_rn(row_buf[c], inv))), inverse));
        return;
    }
    for (int c0 = 0; c0 < n; c0 += 1024) {  // n is a multiple of 128
        const int c = c0 + tid;
        const float b = c < n ? bf16_bits_to_f32(f32_to_bf16_bits(__fmul_rn(row_buf[c], inv))) : 0.0f;
        float m = fabsf(b);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        if (lane == 0) wmax[wave] = m;
        __syncthreads();
        const float bm = fmaxf(wmax[wave & ~1], wmax[wave | 1]);
        const float scale = bm > 0.0f ? __fdiv_rn(bm, 127.0f) : 1.0f;
        const float inverse = __fdiv_rn(1.0f, scale);
        if (c < n) {
            q[static_cast<std::size_t>(r) * n + c] = static_cast<std::int8_t>(quantize_act(b, inverse));
            if (c % 128 == 0) qs[static_cast<std::size_t>(r) * (n / 128) + c / 128] = scale;
        }
        __syncthreads();
    }
}


// y[r, c] = (or +=) the sum of part[q][r][c] over the P parts, in part order (the single-call form of the pass kernels'
// K-parts: Store or Add, any row stride of y).
template <int P, bool ADD>
__global__ void __launch_bounds__(256) parts_sum_kernel(const float* __restrict__ part, int t, int n, float* __restrict__ y,
                                                        std::size_t ld_y) {
    const int per_row = n / 4;
    const int total = t * per_row;
    for (int id = blockIdx.x * 256 + threadIdx.x; id < total; id += gridDim.x * 256) {
        const int r = id / per_row, c = 4 * (id % per_row);
        float4 v[P];
#pragma unroll
        for (int q = 0; q < P; ++q) v[q] = *reinterpret_cast<const float4*>(part + (static_cast<std::size_t>(q) * t + r) * n + c);
        float4 a = v[0];
#pragma unroll
        for (int q = 1; q < P; ++q) {
            a.x = __fadd_rn(a.x, v[q].x);
            a.y = __fadd_rn(a.y, v[q].y);
            a.z = __fadd_rn(a.z, v[q].z);
            a.w = __fadd_rn(a.w, v[q].w);
        }
        float* dst = y + static_cast<std::size_t>(r) * ld_y + c;
        if constexpr (ADD) {
            dst[0] = __fadd_rn(dst[0], a.x);
            dst[1] = __fadd_rn(dst[1], a.y);
            dst[2] = __fadd_rn(dst[2], a.z);
            dst[3] = __fadd_rn(dst[3], a.w);
        } else {
            dst[0] = a.x;
            dst[1] = a.y;
            dst[2] = a.z;
            dst[3] = a.w;
        }
    }
}

} // namespace stack
} // namespace sepal::hip

namespace sepal::hip {

namespace {

int device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        throw LaunchError("small-M stack: device query failed");
    return cus;
}

// LDS of one pass: 16 staged rows of row_bytes (+16 padding), the workers' tile slots, the block's scales, the
// workers' transpose buffers, and the q8 activation scales (16 rows x 24 groups at most)
std::size_t pass_lds(std::size_t row_bytes) {
    return 16 * (row_bytes + 16) + static_cast<std::size_t>(stack::kWorkers) * stack::kSlots * 256 * sizeof(float) +
           static_cast<std::size_t>(stack::kWorkers) * stack::kPairs * 16 * sizeof(float) +
           static_cast<std::size_t>(stack::kWorkers) * 2048 + 16 * 24 * sizeof(float);
}

template <typename Kernel>
void raise_lds(Kernel kernel, std::size_t lds) {
    raise_dynamic_lds(reinterpret_cast<const void*>(kernel), lds, "small-M stack");
}

} // namespace

// The finish pass with the plan's part count as a compile-time constant.
template <int P = 1>
void launch_finish(int parts, std::size_t t, std::size_t hidden, const float* part, float* y, void* xn, double eps,
                   std::int8_t* q, float* qs, int qblock, hipStream_t stream) {
    if constexpr (P < stack::kFinishParts) {
        if (parts != P) {
            launch_finish<P + 1>(parts, t, hidden, part, y, xn, eps, q, qs, qblock, stream);
            return;
        }
    }
    if (parts != P) throw LaunchError("small-M stack: K-part count beyond the finish pass");
    stack::finish_kernel<P><<<dim3(static_cast<unsigned>(t)), dim3(1024), hidden * sizeof(float), stream>>>(
        part, static_cast<int>(t), static_cast<int>(hidden), y, static_cast<std::uint16_t*>(xn), eps, q, qs, qblock);
}

bool small_stack_plan(std::size_t t, std::size_t hidden, std::size_t inter, SmallStackPlan& plan) {
    constexpr std::size_t kLds = 160u << 10;
    constexpr int kMaxPairs = stack::kWorkers * stack::kPairs;  // pairs of one block
    constexpr std::size_t kMaxK = stack::kXChunks * stack::kThreads * 16 / (16 * 2);  // staged X columns
    if (t == 0 || t > 16 || hidden % 128 != 0 || inter % 128 != 0) return false;
    const int g = device_cus();
    const int gh = static_cast<int>(hidden / 128), gi = static_cast<int>(inter / 128);
    // gate/up: whole tiles of 8 features per block over the full K; 8 pairs of a wave touch at most 3 tiles when a
    // tile has >= 4 groups
    const int tiles = static_cast<int>(inter / 8);
    const int per_a = (tiles + g - 1) / g;
    if (gh < 4 || per_a > stack::kWaves || per_a * gh > kMaxPairs || hidden > kMaxK || pass_lds(2 * hidden) > kLds) return false;
    // down: K-parts x blocks of column tiles, at most one block per CU, the fewest pairs per block plus two per part
    // (each part is read back by the finish pass); every part has >= 4 groups
    const int ntile = static_cast<int>((hidden + 15) / 16);
    int best_kp = 0, best_pb = 0, best_cost = 0;
    for (int kp = 1; kp <= stack::kFinishParts && gi / kp >= 4; ++kp) {
        const int gpt = (gi + kp - 1) / kp;
        if (static_cast<std::size_t>(gpt) * 128 > kMaxK || pass_lds(static_cast<std::size_t>(gpt) * 256) > kLds) continue;
        for (int pb = 1; pb <= ntile; ++pb) {
            const int blocks = kp * ((ntile + pb - 1) / pb);
            if (blocks > g) continue;
            if (pb * gpt > kMaxPairs || pb > stack::kWaves) break;
            const int cost = pb * gpt + 2 * kp;  // the pairs of a block, plus the finish pass's reads of the parts
            if (best_kp == 0 || cost < best_cost) {
                best_kp = kp;
                best_pb = pb;
                best_cost = cost;
            }
            break;  // the smallest pb that fits is the cheapest for this kp
        }
    }
    if (best_kp == 0) return false;
    plan.blocks = g;
    plan.tiles_per_block = per_a;
    plan.parts = best_kp;
    plan.units_per_block = best_pb;
    return true;
}

void launch_small_layer(const SmallStackPlan& plan, std::size_t t, std::size_t hidden, std::size_t inter, const void* x,
                        const std::int8_t* w_gu, const float* s_gu, const std::int8_t* w_d, const float* s_d, void* h,
                        float* part, float* y, void* xn, double eps, hipStream_t stream, bool stream_w) {
    using namespace stack;
    // gate/up: x bf16 [t, hidden] -> H binary16 [t, inter]
    PassParams a{};
    a.x = static_cast<const unsigned short*>(x);
    a.ld_x = hidden;
    a.w = reinterpret_cast<const signed char*>(w_gu);
    a.ld_w = hidden;
    a.s = s_gu;
    a.ld_s = hidden / 128;
    a.y = h;
    a.ld_y = inter;
    a.t = static_cast<int>(t);
    a.n = static_cast<int>(2 * inter);
    a.k = static_cast<int>(hidden);
    a.tiles = static_cast<int>(inter / 8);
    a.parts = 1;
    a.per_block = plan.tiles_per_block;
    a.blocks_per_part = (a.tiles + a.per_block - 1) / a.per_block;
    const auto ka = stream_w ? pass_kernel<SEPAL_HIP_BF16, true, SEPAL_HIP_F16, true> : pass_kernel<SEPAL_HIP_BF16, true, SEPAL_HIP_F16>;
    const std::size_t lds_a = pass_lds(2 * hidden);
    raise_lds(ka, lds_a);
    ka<<<dim3(a.blocks_per_part), dim3(kThreads), lds_a, stream>>>(a);
    check_launch("small-M stack gate/up launch");
    // down: H [t, inter] -> P [parts][t][hidden]
    PassParams d{};
    d.x = static_cast<const unsigned short*>(h);
    d.ld_x = inter;
    d.w = reinterpret_cast<const signed char*>(w_d);
    d.ld_w = inter;
    d.s = s_d;
    d.ld_s = inter / 128;
    d.y = part;
    d.ld_y = hidden;
    d.t = static_cast<int>(t);
    d.n = static_cast<int>(hidden);
    d.k = static_cast<int>(inter);
    d.tiles = static_cast<int>((hidden + 15) / 16);
    d.parts = plan.parts;
    d.per_block = plan.units_per_block;
    d.blocks_per_part = (d.tiles + d.per_block - 1) / d.per_block;
    const auto kd = stream_w ? pass_kernel<SEPAL_HIP_F16, false, SEPAL_HIP_F32, true> : pass_kernel<SEPAL_HIP_F16, false, SEPAL_HIP_F32>;
    const std::size_t gpt = (inter / 128 + plan.parts - 1) / plan.parts;
    const std::size_t lds_d = pass_lds(gpt * 256);
    raise_lds(kd, lds_d);
    kd<<<dim3(d.parts * d.blocks_per_part), dim3(kThreads), lds_d, stream>>>(d);
    check_launch("small-M stack down launch");
    // y = sum of the parts; next layer's input
    launch_finish(plan.parts, t, hidden, part, y, xn, eps, nullptr, nullptr, 0, stream);
    check_launch("small-M stack finish launch");
}


void launch_stream_layout(const std::int8_t* w, std::size_t ld_w, std::size_t n, std::size_t k, bool interleave, std::int8_t* out,
                          hipStream_t stream) {
    if (n % 16 != 0 || k % 128 != 0 || n == 0 || k == 0) throw LaunchError("stream layout: n must be a multiple of 16 and k of 128");
    const std::size_t items = n / 16 * (k / 128) * 128;
    stack::stream_layout_kernel<<<dim3(static_cast<unsigned>((items + 255) / 256)), dim3(256), 0, stream>>>(
        reinterpret_cast<const signed char*>(w), ld_w, static_cast<int>(n), static_cast<int>(k), interleave ? 1 : 0,
        reinterpret_cast<signed char*>(out));
    check_launch("stream layout launch");
}

void launch_small_layer_q8(const SmallStackPlan& plan, std::size_t t, std::size_t hidden, std::size_t inter,
                           const std::int8_t* xq, const float* xs, bool per_token, const std::int8_t* w_gu, const float* s_gu,
                           const std::int8_t* w_d, const float* s_d, float* h, float* hmax, float* part, float* y,
                           std::int8_t* xq_next, float* xs_next, void* xn, double eps, hipStream_t stream, bool stream_w) {
    using namespace stack;
    // gate/up: int8 X [t, hidden] (+ scales) -> H [t, inter], float32 per 128 columns, binary16 per token (+ per token:
    // partial row maxima of |H|)
    PassParams a{};
    a.x = reinterpret_cast<const unsigned short*>(xq);
    a.ld_x = hidden;  // bytes
    a.w = reinterpret_cast<const signed char*>(w_gu);
    a.ld_w = hidden;
    a.s = s_gu;
    a.ld_s = hidden / 128;
    a.y = h;
    a.ld_y = inter;
    a.t = static_cast<int>(t);
    a.n = static_cast<int>(2 * inter);
    a.k = static_cast<int>(hidden);
    a.tiles = static_cast<int>(inter / 8);
    a.parts = 1;
    a.per_block = plan.tiles_per_block;
    a.blocks_per_part = (a.tiles + a.per_block - 1) / a.per_block;
    a.xs = xs;
    a.ld_xs = per_token ? 1 : hidden / 128;
    a.per_token = per_token ? 1 : 0;
    a.h16 = per_token ? 1 : 0;
    a.pmax = hmax;
    const auto ka = stream_w ? pass_kernel<kActI8, true, SEPAL_HIP_F32, true> : pass_kernel<kActI8, true, SEPAL_HIP_F32>;
    const std::size_t lds_a = pass_lds(hidden);
    raise_lds(ka, lds_a);
    ka<<<dim3(a.blocks_per_part), dim3(kThreads), lds_a, stream>>>(a);
    check_launch("small-M q8 stack gate/up launch");
    // down: H quantized per block of 128 or per token while staged -> P [parts][t][hidden]
    PassParams d{};
    d.xf = h;
    d.ld_x = inter;
    d.w = reinterpret_cast<const signed char*>(w_d);
    d.ld_w = inter;
    d.s = s_d;
    d.ld_s = inter / 128;
    d.y = part;
    d.ld_y = hidden;
    d.t = static_cast<int>(t);
    d.n = static_cast<int>(hidden);
    d.k = static_cast<int>(inter);
    d.tiles = static_cast<int>((hidden + 15) / 16);
    d.parts = plan.parts;
    d.per_block = plan.units_per_block;
    d.blocks_per_part = (d.tiles + d.per_block - 1) / d.per_block;
    d.per_token = per_token ? 1 : 0;
    d.h16 = per_token ? 1 : 0;
    d.x = reinterpret_cast<const unsigned short*>(h);
    d.hmax = hmax;
    d.hmax_blocks = a.blocks_per_part;

    const auto kd = per_token ? (stream_w ? pass_kernel<kActI8, false, SEPAL_HIP_F32, true, true> : pass_kernel<kActI8, false, SEPAL_HIP_F32, false, true>)
                              : (stream_w ? pass_kernel<kActI8, false, SEPAL_HIP_F32, true> : pass_kernel<kActI8, false, SEPAL_HIP_F32>);
    const std::size_t gpt = (inter / 128 + plan.parts - 1) / plan.parts;
    const std::size_t lds_d = pass_lds(gpt * 128);
    raise_lds(kd, lds_d);
    kd<<<dim3(d.parts * d.blocks_per_part), dim3(kThreads), lds_d, stream>>>(d);
    check_launch("small-M q8 stack down launch");
    // y = sum of the parts; the next layer's bf16 input (xn) and its int8 form
    launch_finish(plan.parts, t, hidden, part, y, xn, eps, xq_next, xs_next, per_token ? static_cast<int>(hidden) : 128,
                  stream);
    check_launch("small-M q8 stack finish launch");
}


// ---- one multiply at M <= 16 on the pass kernels (sepal_hip_gemm_w8g's default for T <= 16) -------------------------

namespace {

template <int P = 1>
void launch_parts_sum(int parts, bool add, std::size_t t, std::size_t n, const float* part, float* y, std::size_t ld_y,
                      hipStream_t stream) {
    if constexpr (P < stack::kFinishParts) {
        if (parts != P) {
            launch_parts_sum<P + 1>(parts, add, t, n, part, y, ld_y, stream);
            return;
        }
    }
    if (parts != P) throw LaunchError("small-M multiply: K-part count beyond the parts sum");
    const int grid = static_cast<int>(std::min<std::size_t>((t * n / 4 + 255) / 256, 1024));
    if (add) stack::parts_sum_kernel<P, true><<<grid, 256, 0, stream>>>(part, static_cast<int>(t), static_cast<int>(n), y, ld_y);
    else stack::parts_sum_kernel<P, false><<<grid, 256, 0, stream>>>(part, static_cast<int>(t), static_cast<int>(n), y, ld_y);
}

template <int XT, bool SWIGLU, int YT, bool STREAM = false>
void launch_pass(const stack::PassParams& p, std::size_t lds, hipStream_t stream) {
    const auto kernel = stack::pass_kernel<XT, SWIGLU, YT, STREAM>;
    raise_lds(kernel, lds);
    kernel<<<dim3(p.parts * p.blocks_per_part), dim3(stack::kThreads), lds, stream>>>(p);
    check_launch("small-M multiply pass launch");
}

// The pass on the packed weights, or on their stream layout when the caller passed that.
template <int XT, bool SWIGLU, int YT>
void launch_pass_w(const GemmArgs& a, const stack::PassParams& p, std::size_t lds, hipStream_t stream) {
    if (a.w_stream) launch_pass<XT, SWIGLU, YT, true>(p, lds, stream);
    else launch_pass<XT, SWIGLU, YT>(p, lds, stream);
}

} // namespace

bool small_gemm_plan(const GemmArgs& a, SmallGemmPlan& plan) {
    constexpr std::size_t kLds = 160u << 10;
    constexpr int kMaxPairs = stack::kWorkers * stack::kPairs;
    constexpr std::size_t kMaxK = stack::kXChunks * stack::kThreads * 16 / (16 * 2);
    if (a.t == 0 || a.t > 16 || (a.x_type != SEPAL_HIP_BF16 && a.x_type != SEPAL_HIP_F16) || a.k % 128 != 0) return false;
    const int g = device_cus();
    const int groups = static_cast<int>(a.k / 128);
    if (a.epilogue == SEPAL_HIP_SWIGLU) {
        // whole tiles (8 features: 8 gate and 8 up rows) over the full K, tiles dealt to one block per CU
        if (a.n % 128 != 0 || groups < 4 || a.k > kMaxK || pass_lds(2 * a.k) > kLds) return false;
        const int tiles = static_cast<int>(a.n / 16);
        const int per = (tiles + g - 1) / g;
        if (per > stack::kWaves || per * groups > kMaxPairs) return false;
        plan.parts = 1;
        plan.per_block = per;
        plan.lds = pass_lds(2 * a.k);
        return true;
    }
    if (a.y_type != SEPAL_HIP_F32 || a.n % 16 != 0) return false;
    // (K-part, 16-column tile) units: the fewest pairs per block (plus the parts sum's reads) within one block per CU
    const int ntile = static_cast<int>(a.n / 16);
    int best_kp = 0, best_pb = 0, best_cost = 0;
    for (int kp = 1; kp <= stack::kFinishParts && groups / kp >= 4; ++kp) {
        const int gpt = (groups + kp - 1) / kp;
        if (static_cast<std::size_t>(gpt) * 128 > kMaxK || pass_lds(static_cast<std::size_t>(gpt) * 256) > kLds) continue;
        if (static_cast<std::size_t>(kp) * a.t * a.n * sizeof(float) > kPartialBytes) break;
        for (int pb = 1; pb <= ntile; ++pb) {
            const int blocks = kp * ((ntile + pb - 1) / pb);
            if (blocks > g) continue;
            if (pb * gpt > kMaxPairs || pb > stack::kWaves) break;
            const int cost = pb * gpt + 2 * kp;
            if (best_kp == 0 || cost < best_cost) {
                best_kp = kp;
                best_pb = pb;
                best_cost = cost;
            }
            break;
        }
    }
    if (best_kp == 0) return false;
    plan.parts = best_kp;
    plan.per_block = best_pb;
    plan.lds = pass_lds(static_cast<std::size_t>((groups + best_kp - 1) / best_kp) * 256);
    return true;
}

bool small_gemm_plan_q8(const GemmArgs& a, SmallGemmPlan& plan) {
    // the q8 gate/up pass (int8 X staged as it is, exact int32 group sums, the cpu-q8 float chain per worker's run of
    // groups): SwiGLU to a float32 H only
    if (a.epilogue != SEPAL_HIP_SWIGLU || a.y_type != SEPAL_HIP_F32) return false;
    GemmArgs b = a;
    b.x_type = SEPAL_HIP_BF16;  // the tile plan does not depend on the activation type
    if (!small_gemm_plan(b, plan)) return false;
    const bool per_token = a.act_block == a.k && a.k != 128;
    // the staged int8 rows (16-byte chunks) and the per-128 scales (16 rows x 24 groups) fit the pass's LDS plan
    return per_token || a.k / 128 <= 24;
}

void launch_small_gemm_q8(const GemmArgs& a, const SmallGemmPlan& plan, hipStream_t stream) {
    using namespace stack;
    if (a.scratch == nullptr) throw LaunchError("small-M multiply: the row maxima need the workspace");
    PassParams p{};
    p.x = static_cast<const unsigned short*>(a.x);
    p.ld_x = a.ld_x;
    p.w = reinterpret_cast<const signed char*>(a.w);
    p.ld_w = a.ld_w;
    p.s = a.s;
    p.ld_s = a.ld_s;
    p.y = a.y;
    p.ld_y = a.ld_y;
    p.t = static_cast<int>(a.t);
    p.n = static_cast<int>(a.n);
    p.k = static_cast<int>(a.k);
    p.parts = 1;
    p.per_block = plan.per_block;
    p.tiles = static_cast<int>(a.n / 16);
    p.blocks_per_part = (p.tiles + p.per_block - 1) / p.per_block;
    p.xs = a.xs;
    p.ld_xs = a.ld_xs;
    p.per_token = a.act_block == a.k && a.k != 128 ? 1 : 0;
    p.pmax = reinterpret_cast<float*>(static_cast<char*>(a.scratch) + kCounterBytes);  // unused by the caller
    launch_pass_w<kActI8, true, SEPAL_HIP_F32>(a, p, plan.lds, stream);
}

bool small_q8_group_sums(const GemmArgs& a, hipStream_t stream) {
    using namespace stack;
    if (a.t == 0 || a.t > 16 || a.scratch == nullptr || a.sums == nullptr) return false;
    // the gate/up pass (its 64-row interleaved tiles) when N is a multiple of 128, else the K-parts pass; no scales
    // are applied (the loaders read a placeholder in the workspace)
    GemmArgs b = a;
    b.x_type = SEPAL_HIP_BF16;
    b.y_type = SEPAL_HIP_F32;
    b.epilogue = a.n % 128 == 0 ? SEPAL_HIP_SWIGLU : SEPAL_HIP_STORE;
    SmallGemmPlan plan;
    if (!small_gemm_plan(b, plan)) {
        if (b.epilogue == SEPAL_HIP_STORE) return false;
        b.epilogue = SEPAL_HIP_STORE;
        if (!small_gemm_plan(b, plan)) return false;
    }
    const bool swiglu = b.epilogue == SEPAL_HIP_SWIGLU;
    if (!swiglu && (a.k / 128 + plan.parts - 1) / plan.parts > 24) return false;
    const float* dummy = reinterpret_cast<const float*>(static_cast<const char*>(a.scratch) + kCounterBytes);
    PassParams p{};
    p.x = static_cast<const unsigned short*>(a.x);
    p.ld_x = a.ld_x;
    p.w = reinterpret_cast<const signed char*>(a.w);
    p.ld_w = a.ld_w;
    p.s = dummy;
    p.ld_s = 0;
    p.t = static_cast<int>(a.t);
    p.n = static_cast<int>(a.n);
    p.k = static_cast<int>(a.k);
    p.parts = plan.parts;
    p.per_block = plan.per_block;
    p.tiles = static_cast<int>(a.n / 16);
    p.blocks_per_part = (p.tiles + p.per_block - 1) / p.per_block;
    p.xs = dummy;
    p.ld_xs = 0;
    p.per_token = 1;
    p.sums = a.sums;
    if (swiglu) launch_pass<kActI8, true, SEPAL_HIP_F32>(p, plan.lds, stream);
    else launch_pass<kActI8X, false, SEPAL_HIP_F32>(p, plan.lds, stream);
    return true;
}

bool small_gemm_plan_q8_parts(const GemmArgs& a, SmallGemmPlan& plan) {
    // one q8 Store / Add multiply: int8 X staged per K-part, the cpu-q8 chain per worker's run of groups, K-parts
    if (a.epilogue == SEPAL_HIP_SWIGLU || a.y_type != SEPAL_HIP_F32) return false;
    GemmArgs b = a;
    b.x_type = SEPAL_HIP_BF16;
    if (!small_gemm_plan(b, plan)) return false;
    const bool per_token = a.act_block == a.k && a.k != 128;
    return per_token || static_cast<std::size_t>((a.k / 128 + plan.parts - 1) / plan.parts) <= 24;
}

void launch_small_gemm_q8_parts(const GemmArgs& a, const SmallGemmPlan& plan, hipStream_t stream) {
    using namespace stack;
    if (a.scratch == nullptr) throw LaunchError("small-M multiply: the K-parts need the workspace");
    float* part = reinterpret_cast<float*>(static_cast<char*>(a.scratch) + kCounterBytes);
    PassParams p{};
    p.x = static_cast<const unsigned short*>(a.x);
    p.ld_x = a.ld_x;
    p.w = reinterpret_cast<const signed char*>(a.w);
    p.ld_w = a.ld_w;
    p.s = a.s;
    p.ld_s = a.ld_s;
    p.y = part;
    p.ld_y = a.n;
    p.t = static_cast<int>(a.t);
    p.n = static_cast<int>(a.n);
    p.k = static_cast<int>(a.k);
    p.parts = plan.parts;
    p.per_block = plan.per_block;
    p.tiles = static_cast<int>(a.n / 16);
    p.blocks_per_part = (p.tiles + p.per_block - 1) / p.per_block;
    p.xs = a.xs;
    p.ld_xs = a.ld_xs;
    p.per_token = a.act_block == a.k && a.k != 128 ? 1 : 0;
    launch_pass_w<kActI8X, false, SEPAL_HIP_F32>(a, p, plan.lds, stream);
    launch_parts_sum(plan.parts, a.epilogue == SEPAL_HIP_ADD, a.t, a.n, part, static_cast<float*>(a.y), a.ld_y, stream);
    check_launch("small-M multiply parts sum launch");
}

void launch_small_gemm_w8g(const GemmArgs& a, const SmallGemmPlan& plan, hipStream_t stream) {
    using namespace stack;
    PassParams p{};
    p.x = static_cast<const unsigned short*>(a.x);
    p.ld_x = a.ld_x;
    p.w = reinterpret_cast<const signed char*>(a.w);
    p.ld_w = a.ld_w;
    p.s = a.s;
    p.ld_s = a.ld_s;
    p.t = static_cast<int>(a.t);
    p.n = static_cast<int>(a.n);
    p.k = static_cast<int>(a.k);
    p.parts = plan.parts;
    p.per_block = plan.per_block;
    if (a.epilogue == SEPAL_HIP_SWIGLU) {
        p.y = a.y;
        p.ld_y = a.ld_y;
        p.tiles = static_cast<int>(a.n / 16);
        p.blocks_per_part = (p.tiles + p.per_block - 1) / p.per_block;
        const bool bf = a.x_type == SEPAL_HIP_BF16;
        switch (a.y_type) {
        case SEPAL_HIP_F32:
            bf ? launch_pass_w<SEPAL_HIP_BF16, true, SEPAL_HIP_F32>(a, p, plan.lds, stream)
               : launch_pass_w<SEPAL_HIP_F16, true, SEPAL_HIP_F32>(a, p, plan.lds, stream);
            break;
        case SEPAL_HIP_BF16:
            bf ? launch_pass_w<SEPAL_HIP_BF16, true, SEPAL_HIP_BF16>(a, p, plan.lds, stream)
               : launch_pass_w<SEPAL_HIP_F16, true, SEPAL_HIP_BF16>(a, p, plan.lds, stream);
            break;
        default:
            bf ? launch_pass_w<SEPAL_HIP_BF16, true, SEPAL_HIP_F16>(a, p, plan.lds, stream)
               : launch_pass_w<SEPAL_HIP_F16, true, SEPAL_HIP_F16>(a, p, plan.lds, stream);
            break;
        }
        return;
    }
    if (a.scratch == nullptr) throw LaunchError("small-M multiply: the K-parts need the workspace");
    float* part = reinterpret_cast<float*>(static_cast<char*>(a.scratch) + kCounterBytes);
    p.y = part;
    p.ld_y = a.n;
    p.tiles = static_cast<int>(a.n / 16);
    p.blocks_per_part = (p.tiles + p.per_block - 1) / p.per_block;
    if (a.x_type == SEPAL_HIP_BF16) launch_pass_w<SEPAL_HIP_BF16, false, SEPAL_HIP_F32>(a, p, plan.lds, stream);
    else launch_pass_w<SEPAL_HIP_F16, false, SEPAL_HIP_F32>(a, p, plan.lds, stream);
    launch_parts_sum(plan.parts, a.epilogue == SEPAL_HIP_ADD, a.t, a.n, part, static_cast<float*>(a.y), a.ld_y, stream);
    check_launch("small-M multiply parts sum launch");
}

} // namespace sepal::hip
