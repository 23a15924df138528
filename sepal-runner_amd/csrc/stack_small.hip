// The M <= 16 layer of the MLP stack (gpu-w8g, and its gpu-q8w form): three launches per layer, no cross-block
// hand-off inside a kernel.
//
// At 16 tokens each layer is a single pass over 77 MB of int8 weights and scales, so the kernels are shaped to keep
// every CU streaming its share of weights for the whole kernel:
//   tiles  (gate/up, SwiGLU): one block of 16 waves per CU, and each block owns whole 16-row weight tiles (8 gate rows
//          and the 8 up rows of the same features) over the full K, 4 or 5 tiles per CU at the model's shape. Every
//          wave first stages one X row in LDS; then 4 loader waves stage the block's scales while the 12 worker waves
//          already have every weight load of their pairs in flight; the block's (tile, group) pairs are split evenly
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

// Activation type of the gpu-q8w stack: int8 X (and int8 H, quantized by the down pass's loaders) on int8 MFMAs.
constexpr int kActI8 = 8;

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
    const float* xf;          // down: H float32 [T, ld_x], quantized here
    const float* hmax;        // down, per token: the gate/up pass's partial row maxima of |H| [T, hmax_blocks]
    int hmax_blocks;
    float* pmax;              // gate/up, per token: this pass's partial row maxima [T, gridDim.x]
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
template <int XT, bool SWIGLU, int YT>
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
    constexpr bool Q8 = XT == kActI8;
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
    // ---- every wave stages one row of X (rows past T repeat row T - 1 and feed only outputs that are never stored)
    // before any weight load is issued: behind a weight burst these loads would wait in the memory queues (M = 16
    // stack: w8g 1.240 -> 1.197 ms per pass; q8 1.46 -> 1.30 ms) ----
    const int xr = min(wave, p.t - 1);
    if constexpr (Q8 && !SWIGLU) {
        // q8 down: H float32 quantized as the activation quantizer does (rule RECIPROCAL, scale = max / 127), per 128
        // columns or with the row maximum of the gate/up pass's partial maxima (per token)
        if (gpt <= 14) stage_h_q8<7, 1>(p, lds, xsc, xpitch, g_lo, gpt, wave, 1, lane);
        else stage_h_q8<12, 1>(p, lds, xsc, xpitch, g_lo, gpt, wave, 1, lane);
    } else if constexpr (Q8) {
        // q8 gate/up: int8 rows (16-byte chunks of 16 columns) and the rows' activation scales
        const int cq = kw / 16;
        const unsigned char* xrow = reinterpret_cast<const unsigned char*>(p.x) + static_cast<std::size_t>(xr) * p.ld_x + 128 * g_lo;
        u32x4 xv[kXChunks / 2];
#pragma unroll
        for (int e = 0; e < kXChunks / 2; ++e) xv[e] = *reinterpret_cast<const u32x4*>(xrow + 16 * min(lane + 64 * e, cq - 1));
        const int nsc = p.per_token ? 1 : gpt;
        const float xsv = p.xs[static_cast<std::size_t>(xr) * p.ld_xs + (p.per_token ? 0 : g_lo + min(lane, nsc - 1))];
#pragma unroll
        for (int e = 0; e < kXChunks / 2; ++e)
            if (lane + 64 * e < cq) *reinterpret_cast<u32x4*>(lds + wave * xpitch + 16 * (lane + 64 * e)) = xv[e];
        if (lane < nsc) xsc[p.per_token ? wave : wave * gpt + lane] = xsv;
    } else {
        const int cpr = kw / 8;
        const unsigned short* xrow = p.x + static_cast<std::size_t>(xr) * p.ld_x + 128 * g_lo;
        u32x4 xv[kXChunks];
#pragma unroll
        for (int e = 0; e < kXChunks; ++e) xv[e] = *reinterpret_cast<const u32x4*>(xrow + 8 * min(lane + 64 * e, cpr - 1));
#pragma unroll
        for (int e = 0; e < kXChunks; ++e)
            if (lane + 64 * e < cpr) *reinterpret_cast<u32x4*>(lds + wave * xpitch + 16 * (lane + 64 * e)) = xv[e];
    }
    __syncthreads();

    if (wave < kLoaders) {
        // ---- loaders: the block's weight scales (row runs of gpt words) ----
        const int lt = tid;      // 0 .. 64 kLoaders - 1
        float sv[kScaleLoads];
#pragma unroll
        for (int e = 0; e < kScaleLoads; ++e) {
            const int idx = min(lt + e * 64 * kLoaders, total * 16 - 1);
            const int tl = idx / (16 * gpt), rem = idx % (16 * gpt);
            const int row = min(tile_row<SWIGLU>(tile0 + tl, rem / gpt), p.n - 1);
            sv[e] = p.s[static_cast<std::size_t>(row) * p.ld_s + g_lo + rem % gpt];
        }
#pragma unroll
        for (int e = 0; e < kScaleLoads; ++e)
            if (lt + e * 64 * kLoaders < total * 16) scl[lt + e * 64 * kLoaders] = sv[e];
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
                const signed char* src = wrow[0] + 128 * g;
#pragma unroll
                for (int j = 1; j < kSlots; ++j)
                    if (slot == j) src = wrow[j] + 128 * g;
                wb[i][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
                wb[i][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + kRowStep * p.ld_w));
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
            const int q = q0 + i;
            if (i > 0 && q % gpt == 0) {  // a new tile (wave-uniform)
                flush(cur_slot);
                ++cur_slot;
                cur = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
            const float sc = scl[((first_tile + pslot[i]) * 16 + lane % 16) * gpt + (pg[i] - g_lo)];
            const int kofs = 128 * (q % gpt);
            f32x4 prt = {0.0f, 0.0f, 0.0f, 0.0f};
            *reinterpret_cast<u32x4*>(tb + wr_lo) = wb[i][0];
            *reinterpret_cast<u32x4*>(tb + wr_hi) = wb[i][1];
            if constexpr (Q8) {
                // the int8 weights go to the MFMA as they are: the exact int32 group sum, then the cpu-q8 float chain
                // (runner/src/cpu/gemm_kernels_avx512.cpp:67-115): t = fma(f_g, ws_g, t) with one scale per token
                // (applied after the sum), fma(f_g, ws_g * xs_g, t) with one per 128 columns
                i32x4 acc = {0, 0, 0, 0};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int rr = lane % 16, cc = 4 * h + lane / 16;
                    const u32x4 wv = *reinterpret_cast<const u32x4*>(tb + rr * 128 + ((cc + rr / 2) % 8) * 16);
                    const u32x4 a = *reinterpret_cast<const u32x4*>(lds + (lane % 16) * xpitch + kofs + 64 * h + 16 * (lane / 16));
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, wv), acc, 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float s_r = p.per_token ? sc : __fmul_rn(sc, xsc[(4 * (lane / 16) + r) * gpt + q % gpt]);
                    cur[r] = __builtin_fmaf(static_cast<float>(acc[r]), s_r, cur[r]);
                }
                continue;
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int rr = lane % 16, cc = 4 * h + lane / 16;
                const u32x4 wv = *reinterpret_cast<const u32x4*>(tb + rr * 128 + ((cc + rr / 2) % 8) * 16);
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
        // H = swiglu_cephes(gate, up) in float32 (the gpu-q8w epilogue), and, per token, this block's row maxima of |H|
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
            const float hv = swiglu_cephes(g, u);
            hy[static_cast<std::size_t>(r) * p.ld_y + f] = hv;
            if (p.per_token) atomicMax(&row_max[r], __float_as_uint(fabsf(hv)));
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

// y[r][c] = sum over parts (in order) of P[part][r][c]; then, if xn is set, xn[r] = bf16(RMSNorm(y[r])) with the
// cpu-q8 summation order (runner/src/cpu/elementwise.cpp:22-59) and eps. One block of 1024 threads per row; each
// thread's partial loads (up to kFinishParts) are all in flight at once.
constexpr int kFinishParts = 16;

// With q set (the gpu-q8w stack), the bf16 values are also quantized as quantize_rows does (rule RECIPROCAL), with
// one scale per row (qblock = n) or per 128 columns (qblock = 128), into q [t, n] and qs [t, n / qblock].
__global__ void __launch_bounds__(1024) finish_kernel(const float* __restrict__ part, int parts, int t, int n, float* __restrict__ y,
                                                      std::uint16_t* __restrict__ xn, double eps, std::int8_t* __restrict__ q,
                                                      float* __restrict__ qs, int qblock) {
    extern __shared__ __align__(16) float row_buf[];  // [n]
    const int r = blockIdx.x, tid = threadIdx.x;
    for (int c4 = tid; c4 < n / 4; c4 += 1024) {
        float4 v[kFinishParts];
#pragma unroll
        for (int q = 0; q < kFinishParts; ++q)
            v[q] = *reinterpret_cast<const float4*>(part + (static_cast<std::size_t>(min(q, parts - 1)) * t + r) * n + 4 * c4);
        float4 a = v[0];
#pragma unroll
        for (int q = 1; q < kFinishParts; ++q)
            if (q < parts) {
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
            // eight reads in flight, then their eight links of the chain, in order (one read at a time left the wave
            // waiting on LDS latency at every link)
            int c = 0;
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


// ---- the persistent form: one cooperative launch runs every layer ----------------------------------------------------
//
// One block per CU for the whole stack. Per layer: phase A (gate/up -> H), grid barrier, phase B (down -> P, and the
// last block of each column tile adds its K-parts into y), grid barrier, phase C (16 waves make the next layer's X rows,
// bf16(RMSNorm(y))), grid barrier. The phases do the same arithmetic in the same order as pass_kernel and
// finish_kernel, with the same plan, so the results are the same bits. The loader waves do all the hand-offs (staging,
// epilogues, barriers); the workers only stream weights and multiply, and with `early` set they issue the next phase's
// weight loads as soon as their registers are free, so the weights stay in flight across the barriers.
constexpr int kMaxLayers = 64;         // layers of one launch (the host splits longer stacks)
constexpr int kNormHalf = 48;          // row values per lane of the phase-C RMSNorm: 3072 columns at most
constexpr unsigned kSpinLimit = 1u << 16;  // grid-barrier polls before a wait gives up (about 50 ms)

struct StackParams {
    const signed char* w_gu[kMaxLayers];
    const float* s_gu[kMaxLayers];
    const signed char* w_d[kMaxLayers];
    const float* s_d[kMaxLayers];
    unsigned short* x;     // bf16 [t, hidden]: layer 0's input; receives every later layer's input
    unsigned short* h;     // binary16 [t, inter]
    float* part;           // float32 [parts][t][hidden]
    float* y;              // float32 [t, hidden]
    unsigned* tile_count;  // [hidden / 16] arrivals per down column tile, zero at rest
    unsigned* grid_count;  // [3] barrier arrivals and block exits (zero at rest), launches that timed out
    unsigned* timeout;     // set to 1 when a barrier wait gives up (cleared by the launch's last block out)
    double eps;
    int layers, t, hidden, inter;
    int per_a;                // gate/up tiles per block
    int parts, per_d, bpp_d;  // down K-parts, column tiles per block, blocks per part
    int x_region;             // bytes of the staged-row region (16 rows at the widest pitch)
    int early;                // workers issue the next phase's weights before its barrier
};

// Data that one block writes and blocks on other XCDs read (H, P, y, x) is written and read at device coherence (the
// SC1 cache-policy bit on buffer accesses, agent-scope relaxed atomics on plain stores); a writer waits for its stores
// to complete before it arrives at a barrier or counter. No release/acquire fences: on this part they write back and
// invalidate the whole L2.
constexpr int kCoherent = 16;

// A buffer resource over `bytes` bytes at p: loads take one lane offset register, the uniform rest in the scalar
// offset, and reads past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, std::size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}

// The (tile, group) work of one block in one phase: tiles tile0 .. tile0 + ntiles - 1, groups g_lo .. g_lo + gpt - 1,
// total = ntiles * gpt pairs dealt to the workers in runs of `per`.
struct Geo {
    int tile0, ntiles, g_lo, gpt, total, per, part;
};

__device__ __forceinline__ Geo geo_gate_up(const StackParams& p, int b) {
    Geo g;
    g.tile0 = b * p.per_a;
    g.ntiles = max(0, min(p.per_a, p.inter / 8 - g.tile0));
    g.g_lo = 0;
    g.gpt = p.hidden / 128;
    g.part = 0;
    g.total = g.ntiles * g.gpt;
    g.per = (g.total + kWorkers - 1) / kWorkers;
    return g;
}

__device__ __forceinline__ Geo geo_down(const StackParams& p, int b) {
    Geo g;
    const int gi = p.inter / 128;
    g.part = b / p.bpp_d;
    g.tile0 = (b % p.bpp_d) * p.per_d;
    g.ntiles = g.part < p.parts ? max(0, min(p.per_d, p.hidden / 16 - g.tile0)) : 0;
    const int part = min(g.part, p.parts - 1);
    g.g_lo = part * gi / p.parts;
    g.gpt = (part + 1) * gi / p.parts - g.g_lo;
    g.total = g.ntiles * g.gpt;
    g.per = (g.total + kWorkers - 1) / kWorkers;
    return g;
}

// A worker's weight loads of one phase (as pass_kernel: two instructions of 8 rows x 128 bytes per pair; past the
// worker's share the loads stay on its last pair). The row offset within a pair is one lane term; the rest is uniform.
template <bool SWIGLU>
__device__ __forceinline__ void issue_pairs(const Geo& g, const signed char* w, int ld_w, int rows, int wk, int lane,
                                            u32x4 (&wb)[kPairs][2]) {
    if (g.total == 0) return;
    constexpr int kRowStep = SWIGLU ? 64 : 8;
    (void)rows;
    const int q0 = min(wk * g.per, g.total - 1), q1 = min(wk * g.per + g.per, g.total);
    const int qlast = max(q1 - 1, q0);
    const int voff = (lane / 8) * ld_w + 16 * (lane % 8);
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
        const int q = min(q0 + i, qlast);
        const int tile = g.tile0 + q / g.gpt, grp = g.g_lo + q % g.gpt;
        // global loads (a buffer load here would make the compiler wait for every load before the first LDS read)
        const signed char* base = w + static_cast<std::size_t>(tile_row<SWIGLU>(tile, 0)) * ld_w + 128 * grp;
        wb[i][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + voff));
        wb[i][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + voff + kRowStep * ld_w));
    }
}

// A worker's multiply of one phase (the same steps as pass_kernel's workers).
template <int XT>
__device__ __forceinline__ void multiply_pairs(const Geo& g, const unsigned char* xs, int xpitch, float* red, const float* scl,
                                               unsigned char* tb, int wk, int lane, const u32x4 (&wb)[kPairs][2]) {
    const int q0 = min(wk * g.per, g.total), q1 = min(q0 + g.per, g.total);
    const int n_pairs = q1 - q0;
    if (n_pairs <= 0) return;
    const int wr_lo = (lane / 8) * 128 + ((lane % 8 + lane / 16) % 8) * 16;
    const int wr_hi = (8 + lane / 8) * 128 + ((lane % 8 + 4 + lane / 16) % 8) * 16;
    f32x4 cur = {0.0f, 0.0f, 0.0f, 0.0f};
    int cur_slot = 0;
    const auto flush = [&](int slot_) {
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wk * kSlots + slot_) * 256 + (4 * (lane / 16) + r) * 16 + lane % 16] = cur[r];
    };
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
        if (i >= n_pairs) continue;
        const int q = q0 + i;
        if (i > 0 && q % g.gpt == 0) {
            flush(cur_slot);
            ++cur_slot;
            cur = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        const float sc = scl[((q / g.gpt) * 16 + lane % 16) * g.gpt + q % g.gpt];
        const int kofs = 128 * (q % g.gpt);
        f32x4 prt = {0.0f, 0.0f, 0.0f, 0.0f};
        *reinterpret_cast<u32x4*>(tb + wr_lo) = wb[i][0];
        *reinterpret_cast<u32x4*>(tb + wr_hi) = wb[i][1];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int rr = lane % 16, cc = 4 * h + lane / 16;
            const u32x4 wv = *reinterpret_cast<const u32x4*>(tb + rr * 128 + ((cc + rr / 2) % 8) * 16);
            unsigned o[8];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                if constexpr (XT == SEPAL_HIP_BF16) s8x4_to_bf16x4(wv[c], o[2 * c], o[2 * c + 1]);
                else s8x4_to_f16x4(wv[c], o[2 * c], o[2 * c + 1]);
            }
            const unsigned char* xr = xs + (lane % 16) * xpitch + 2 * (kofs + 64 * h + 16 * (lane / 16));
            const u32x4 a0 = *reinterpret_cast<const u32x4*>(xr);
            const u32x4 a1 = *reinterpret_cast<const u32x4*>(xr + 16);
            prt = mfma16(XT, a0, u32x4{o[0], o[1], o[2], o[3]}, prt);
            prt = mfma16(XT, a1, u32x4{o[4], o[5], o[6], o[7]}, prt);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) cur[r] = __builtin_fmaf(prt[r], sc, cur[r]);
    }
    flush(cur_slot);
}

// A loader thread's share of one phase's scales (lt = 0 .. 64 kLoaders - 1), held in registers until the phase's
// staging writes them to LDS.
template <bool SWIGLU>
__device__ __forceinline__ void load_scales(const Geo& g, const float* s, int ld_s, int lt, float (&sv)[kScaleLoads]) {
    if (g.total == 0) return;
#pragma unroll
    for (int e = 0; e < kScaleLoads; ++e) {
        const int idx = min(lt + e * 64 * kLoaders, g.total * 16 - 1);
        const int tl = idx / (16 * g.gpt), rem = idx % (16 * g.gpt);
        sv[e] = s[static_cast<std::size_t>(tile_row<SWIGLU>(g.tile0 + tl, rem / g.gpt)) * ld_s + g.g_lo + rem % g.gpt];
    }
}

// The four loader waves meet (LDS arrival counter; `gen` counts the meetings of this thread).
__device__ __forceinline__ void loaders_meet(unsigned* ctr, unsigned& gen, int lane) {
    gen += kLoaders;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's global stores and LDS writes are done
    if (lane == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    while (__hip_atomic_load(ctr, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < gen) __builtin_amdgcn_s_sleep(1);
}

// Grid barrier number `n` (0-based) of this launch, run by the loaders: every loader wave's stores complete
// (loaders_meet waits for them), then thread 0 arrives and polls with agent-scope relaxed atomics; the other loader
// waves wait in the second loaders_meet. A poll that runs past kSpinLimit (or sees another block's timeout) gives up and sets the timeout flag,
// so every wave still reaches the end of the kernel.
__device__ __forceinline__ void grid_barrier(const StackParams& p, unsigned n, unsigned* ctr, unsigned& gen, int tid, int lane) {
    loaders_meet(ctr, gen, lane);
    if (tid == 0) {
        const unsigned target = (n + 1) * gridDim.x;
        __hip_atomic_fetch_add(&p.grid_count[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (unsigned spin = 0; __hip_atomic_load(&p.grid_count[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target; ++spin) {
            if (spin > kSpinLimit || __hip_atomic_load(p.timeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
                __hip_atomic_store(p.timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    loaders_meet(ctr, gen, lane);
}

// Rows 4 w .. 4 w + 3 (w = loader wave) of a [t, ld] 16-bit matrix, columns col0 .. col0 + kw - 1, into the staged
// rows (rows past T repeat row T - 1), as pass_kernel's loaders.
__device__ __forceinline__ void stage_rows(const unsigned short* src, int ld, int col0, int kw, int t, unsigned char* xs,
                                           int xpitch, int wave, int lane) {
    const int cpr = kw / 8;
#pragma unroll
    for (int rr = 0; rr < 4; rr += 2) {
        u32x4 xv[2][kXChunks];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const __amdgpu_buffer_rsrc_t rr_ = rsrc(src + static_cast<std::size_t>(min(4 * wave + rr + h, t - 1)) * ld + col0, 2 * kw);
#pragma unroll
            for (int e = 0; e < kXChunks; ++e)
                xv[h][e] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rr_, 16 * lane, 1024 * e, kCoherent));
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < kXChunks; ++e)
                if (lane + 64 * e < cpr) *reinterpret_cast<u32x4*>(xs + (4 * wave + rr + h) * xpitch + 16 * (lane + 64 * e)) = xv[h][e];
    }
}

__global__ void __launch_bounds__(kThreads) stack_kernel(const StackParams p) {
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ unsigned ready, done, meet, go;
    __shared__ int is_last[kWaves];
    const int tid = threadIdx.x, lane = tid % 64, b = blockIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);  // uniform: the buffer resources built from it stay scalar
    float* red = reinterpret_cast<float*>(lds + p.x_region);
    float* scl = red + kWorkers * kSlots * 256;
    unsigned char* tbuf = reinterpret_cast<unsigned char*>(scl + kWorkers * kPairs * 16);
    if (tid == 0) {
        ready = 0u;
        done = 0u;
        meet = 0u;
        go = 0u;
    }
    __syncthreads();
    const int xpitch_a = 2 * p.hidden + 16;

    if (wave >= kLoaders) {
        // ---- workers ----
        const int wk = wave - kLoaders;
        unsigned char* tb = tbuf + wk * 2048;
        u32x4 wb[kPairs][2];
        unsigned ph = 0;
        const auto wait_ready = [&]() {
            while (__hip_atomic_load(&ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < kLoaders * (ph + 1))
                __builtin_amdgcn_s_sleep(1);
        };
        const auto wait_go = [&]() {  // the loaders have started the phase (its barrier is behind them)
            while (__hip_atomic_load(&go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < kLoaders * (ph + 1))
                __builtin_amdgcn_s_sleep(1);
        };
        const auto signal_done = [&]() {
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
            if (lane == 0) __hip_atomic_fetch_add(&done, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            ++ph;
        };
        issue_pairs<true>(geo_gate_up(p, b), p.w_gu[0], p.hidden, 2 * p.inter, wk, lane, wb);
        for (int l = 0; l < p.layers; ++l) {
            // the geometry is recomputed per layer from an opaque block index: held across the loop, its per-pair
            // addresses would not fit in registers
            int bl = b;
            asm volatile("" : "+s"(bl));
            const Geo ga = geo_gate_up(p, bl), gd = geo_down(p, bl);
            const int xpitch_d = 2 * 128 * gd.gpt + 16;
            if (!p.early && l > 0) {
                wait_go();
                issue_pairs<true>(ga, p.w_gu[l], p.hidden, 2 * p.inter, wk, lane, wb);
            }
            wait_ready();
            multiply_pairs<SEPAL_HIP_BF16>(ga, lds, xpitch_a, red, scl, tb, wk, lane, wb);
            signal_done();
            if (p.early) issue_pairs<false>(gd, p.w_d[l], p.inter, p.hidden, wk, lane, wb);
            if (!p.early) {
                wait_go();
                issue_pairs<false>(gd, p.w_d[l], p.inter, p.hidden, wk, lane, wb);
            }
            wait_ready();
            multiply_pairs<SEPAL_HIP_F16>(gd, lds, xpitch_d, red, scl, tb, wk, lane, wb);
            signal_done();
            if (p.early && l + 1 < p.layers) issue_pairs<true>(ga, p.w_gu[l + 1], p.hidden, 2 * p.inter, wk, lane, wb);
        }
        return;
    }

    // ---- loaders: lt = 0 .. 255 ----
    const int lt = tid;
    unsigned gen = 0, nbar = 0, ph = 0;
    float sv[kScaleLoads];
    const auto start = [&]() {
        if (lane == 0) __hip_atomic_fetch_add(&go, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
    const auto publish = [&](const Geo& g) {  // the phase's scales to LDS, then the ready flag
#pragma unroll
        for (int e = 0; e < kScaleLoads; ++e)
            if (lt + e * 64 * kLoaders < g.total * 16) scl[lt + e * 64 * kLoaders] = sv[e];
        __builtin_amdgcn_s_waitcnt(0xC07F);
        if (lane == 0) __hip_atomic_fetch_add(&ready, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
    const auto wait_done = [&]() {
        ++ph;
        while (__hip_atomic_load(&done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < kWorkers * ph) __builtin_amdgcn_s_sleep(1);
    };
    // the tile's sum in worker order (as pass_kernel)
    const auto sum_tile = [&](const Geo& g, int tl, int e) {
        const int lo = tl * g.gpt / g.per, hi = ((tl + 1) * g.gpt - 1) / g.per;
        float v = red[(lo * kSlots + (tl - min(lo * g.per, g.total - 1) / g.gpt)) * 256 + e];
        for (int w = lo + 1; w <= hi; ++w) v = __fadd_rn(v, red[(w * kSlots + (tl - min(w * g.per, g.total - 1) / g.gpt)) * 256 + e]);
        return v;
    };
    load_scales<true>(geo_gate_up(p, b), p.s_gu[0], p.hidden / 128, lt, sv);
    for (int l = 0; l < p.layers; ++l) {
        int bl = b;  // opaque per layer, as the workers'
        asm volatile("" : "+s"(bl));
        const Geo ga = geo_gate_up(p, bl), gd = geo_down(p, bl);
        const int xpitch_d = 2 * 128 * gd.gpt + 16;
        // ---- A: gate/up over X (staged from x) -> H ----
        start();
        stage_rows(p.x, p.hidden, 0, p.hidden, p.t, lds, xpitch_a, wave, lane);
        publish(ga);
        load_scales<false>(gd, p.s_d[l], p.inter / 128, lt, sv);
        wait_done();
        for (int id = lt; id < ga.ntiles * 128; id += 64 * kLoaders) {
            const int tl = id / 128, r = (id / 8) % 16, i = id % 8;
            const int tile = ga.tile0 + tl;
            const int f = 64 * (tile / 8) + 8 * (tile % 8) + i;
            if (r >= p.t) continue;
            const float gv = sum_tile(ga, tl, r * 16 + i), uv = sum_tile(ga, tl, r * 16 + 8 + i);
            __hip_atomic_store(p.h + static_cast<std::size_t>(r) * p.inter + f, f32_to_f16_bits(swiglu_fast(gv, uv)),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        grid_barrier(p, nbar++, &meet, gen, tid, lane);
        // ---- B: down over H -> P[part]; the last block of a column tile adds the parts into y ----
        start();
        stage_rows(p.h, p.inter, 128 * gd.g_lo, 128 * gd.gpt, p.t, lds, xpitch_d, wave, lane);
        publish(gd);
        if (l + 1 < p.layers) load_scales<true>(ga, p.s_gu[l + 1], p.hidden / 128, lt, sv);
        wait_done();
        for (int id = lt; id < gd.ntiles * 256; id += 64 * kLoaders) {
            const int tl = id / 256, r = (id / 16) % 16, c = id % 16;
            if (r >= p.t) continue;
            const int col = 16 * (gd.tile0 + tl) + c;
            __hip_atomic_store(&p.part[(static_cast<std::size_t>(gd.part) * p.t + r) * p.hidden + col], sum_tile(gd, tl, r * 16 + c),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        loaders_meet(&meet, gen, lane);
        if (lt < gd.ntiles)
            is_last[lt] = __hip_atomic_fetch_add(&p.tile_count[gd.tile0 + lt], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                          static_cast<unsigned>(p.parts - 1);
        loaders_meet(&meet, gen, lane);
        const __amdgpu_buffer_rsrc_t pres = rsrc(p.part, static_cast<std::size_t>(p.parts) * p.t * p.hidden * 4);
        for (int id = lt; id < gd.ntiles * 256; id += 64 * kLoaders) {
            const int tl = id / 256, r = (id / 16) % 16, c = id % 16;
            if (!is_last[tl] || r >= p.t) continue;
            const int col = 16 * (gd.tile0 + tl) + c;
            const int step = p.t * p.hidden * 4;
            float pv[kFinishParts];
#pragma unroll
            for (int q = 0; q < kFinishParts; ++q)
                pv[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pres, 4 * (r * p.hidden + col), min(q, p.parts - 1) * step, kCoherent));
            float v = pv[0];
#pragma unroll
            for (int q = 1; q < kFinishParts; ++q)
                if (q < p.parts) v = __fadd_rn(v, pv[q]);
            __hip_atomic_store(&p.y[static_cast<std::size_t>(r) * p.hidden + col], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (lt < gd.ntiles && is_last[lt]) __hip_atomic_store(&p.tile_count[gd.tile0 + lt], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (l + 1 == p.layers) break;
        grid_barrier(p, nbar++, &meet, gen, tid, lane);
        // ---- C: x[r] = bf16(RMSNorm(y[r])), one row per wave of blocks 0 .. ceil(t / 4) - 1 (cpu-q8 order: lane
        // L = lane % 32 is accumulator lane L of runner/src/cpu/elementwise.cpp:22-59 and adds c = L, L + 32, ... in
        // order; the upper half-wave holds the second half of the row and continues the lower half's sums) ----
        const int r = 4 * b + wave;
        if (r < p.t) {
            const int L = lane % 32, half = lane / 32, jh = p.hidden / 64;
            const __amdgpu_buffer_rsrc_t yres = rsrc(p.y + static_cast<std::size_t>(r) * p.hidden, 4 * p.hidden);
            const int vo = 4 * (L + 32 * jh * half);
            // all loads unconditional (past the row they read zero; values past jh are never used)
            float v[kNormHalf];
#pragma unroll
            for (int j = 0; j < kNormHalf; ++j) v[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(yres, vo, 128 * j, kCoherent));
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < kNormHalf; ++j) acc = j < jh ? __builtin_fmaf(v[j], v[j], acc) : acc;
            float acc2 = __shfl(acc, L);
#pragma unroll
            for (int j = 0; j < kNormHalf; ++j) acc2 = j < jh ? __builtin_fmaf(v[j], v[j], acc2) : acc2;
            const int l8 = L % 8;
            const float a0 = __shfl(acc2, 32 + l8), a1 = __shfl(acc2, 40 + l8), a2 = __shfl(acc2, 48 + l8),
                        a3 = __shfl(acc2, 56 + l8);
            const float sl = __fadd_rn(__fadd_rn(a0, a1), __fadd_rn(a2, a3));
            const float sl4 = __shfl(sl, (l8 + 4) % 8);
            const float hs = __fadd_rn(sl, sl4);
            const float h0 = __shfl(hs, 0), h1 = __shfl(hs, 1), h2 = __shfl(hs, 2), h3 = __shfl(hs, 3);
            const float sum = __fadd_rn(__fadd_rn(h0, h2), __fadd_rn(h1, h3));
            const float inv = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(sum) / static_cast<double>(p.hidden) + p.eps));
            const __amdgpu_buffer_rsrc_t xres = rsrc(p.x + static_cast<std::size_t>(r) * p.hidden, 2 * p.hidden);
#pragma unroll
            for (int j = 0; j < kNormHalf; ++j)
                if (j < jh) __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(__fmul_rn(v[j], inv)), xres, vo / 2, 64 * j, kCoherent);
        }
        grid_barrier(p, nbar++, &meet, gen, tid, lane);
    }
    // the last block out clears the barrier counters for the next launch
    if (tid == 0 && __hip_atomic_fetch_add(&p.grid_count[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1) {
        __hip_atomic_store(&p.grid_count[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&p.grid_count[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // a timeout is counted (grid_count[2]) and cleared, so the next launch waits normally
        if (__hip_atomic_load(p.timeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
            __hip_atomic_fetch_add(&p.grid_count[2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p.timeout, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
void raise_lds(Kernel kernel, std::size_t lds, std::size_t& raised) {
    if (lds > raised) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(lds)) != hipSuccess)
            throw LaunchError("small-M stack: hipFuncSetAttribute(MaxDynamicSharedMemorySize) failed");
        raised = lds;
    }
}

} // namespace

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
                        float* part, float* y, void* xn, double eps, hipStream_t stream) {
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
    const auto ka = pass_kernel<SEPAL_HIP_BF16, true, SEPAL_HIP_F16>;
    static std::size_t raised_a = 0;
    const std::size_t lds_a = pass_lds(2 * hidden);
    raise_lds(ka, lds_a, raised_a);
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
    const auto kd = pass_kernel<SEPAL_HIP_F16, false, SEPAL_HIP_F32>;
    static std::size_t raised_d = 0;
    const std::size_t gpt = (inter / 128 + plan.parts - 1) / plan.parts;
    const std::size_t lds_d = pass_lds(gpt * 256);
    raise_lds(kd, lds_d, raised_d);
    kd<<<dim3(d.parts * d.blocks_per_part), dim3(kThreads), lds_d, stream>>>(d);
    check_launch("small-M stack down launch");
    // y = sum of the parts; next layer's input
    finish_kernel<<<dim3(static_cast<unsigned>(t)), dim3(1024), hidden * sizeof(float), stream>>>(
        part, plan.parts, static_cast<int>(t), static_cast<int>(hidden), y, static_cast<std::uint16_t*>(xn), eps, nullptr,
        nullptr, 0);
    check_launch("small-M stack finish launch");
}


void launch_small_layer_q8(const SmallStackPlan& plan, std::size_t t, std::size_t hidden, std::size_t inter,
                           const std::int8_t* xq, const float* xs, bool per_token, const std::int8_t* w_gu, const float* s_gu,
                           const std::int8_t* w_d, const float* s_d, float* h, float* hmax, float* part, float* y,
                           std::int8_t* xq_next, float* xs_next, void* xn, double eps, hipStream_t stream) {
    using namespace stack;
    // gate/up: int8 X [t, hidden] (+ scales) -> H float32 [t, inter] (+ per token: partial row maxima of |H|)
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
    a.pmax = hmax;
    const auto ka = pass_kernel<kActI8, true, SEPAL_HIP_F32>;
    static std::size_t raised_a = 0;
    const std::size_t lds_a = pass_lds(hidden);
    raise_lds(ka, lds_a, raised_a);
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
    d.hmax = hmax;
    d.hmax_blocks = a.blocks_per_part;

    const auto kd = pass_kernel<kActI8, false, SEPAL_HIP_F32>;
    static std::size_t raised_d = 0;
    const std::size_t gpt = (inter / 128 + plan.parts - 1) / plan.parts;
    const std::size_t lds_d = pass_lds(gpt * 128);
    raise_lds(kd, lds_d, raised_d);
    kd<<<dim3(d.parts * d.blocks_per_part), dim3(kThreads), lds_d, stream>>>(d);
    check_launch("small-M q8 stack down launch");
    // y = sum of the parts; the next layer's bf16 input (xn) and its int8 form
    finish_kernel<<<dim3(static_cast<unsigned>(t)), dim3(1024), hidden * sizeof(float), stream>>>(
        part, plan.parts, static_cast<int>(t), static_cast<int>(hidden), y, static_cast<std::uint16_t*>(xn), eps, xq_next,
        xs_next, per_token ? static_cast<int>(hidden) : 128);
    check_launch("small-M q8 stack finish launch");
}

bool launch_small_stack(const SmallStackPlan& plan, std::size_t layers, std::size_t t, std::size_t hidden, std::size_t inter,
                        void* x, const std::int8_t* const* w_gu, const float* const* s_gu, const std::int8_t* const* w_d,
                        const float* const* s_d, void* h, float* part, float* y, unsigned* counters, double eps,
                        bool early, hipStream_t stream) {
    using namespace stack;
    const std::size_t gpt_d = (inter / 128 + plan.parts - 1) / plan.parts;
    const std::size_t xr = 16 * std::max(2 * hidden + 16, 2 * 128 * gpt_d + 16);
    const std::size_t lds = pass_lds(0) - 16 * 16 + xr;
    // one block per CU, all resident at once: the kernel's grid barriers need every block running
    static std::size_t raised = 0;
    raise_lds(stack_kernel, lds, raised);
    int dev = 0, coop = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(stack_kernel), kThreads, lds) != hipSuccess)
        throw LaunchError("small-M stack: cooperative-launch query failed");
    if (coop == 0 || per_cu < 1) return false;
    StackParams p{};
    p.x = static_cast<unsigned short*>(x);
    p.h = static_cast<unsigned short*>(h);
    p.part = part;
    p.y = y;
    p.tile_count = counters;
    p.grid_count = counters + 4096;
    p.timeout = counters + 4096 + 3;
    p.eps = eps;
    p.t = static_cast<int>(t);
    p.hidden = static_cast<int>(hidden);
    p.inter = static_cast<int>(inter);
    p.per_a = plan.tiles_per_block;
    p.parts = plan.parts;
    p.per_d = plan.units_per_block;
    p.bpp_d = static_cast<int>((hidden / 16 + plan.units_per_block - 1) / plan.units_per_block);
    p.x_region = static_cast<int>(xr);
    p.early = early ? 1 : 0;
    for (std::size_t l0 = 0; l0 < layers; l0 += kMaxLayers) {
        const std::size_t n = std::min<std::size_t>(kMaxLayers, layers - l0);
        if (l0 > 0) {
            // the previous launch ended after its last down pass: its y and parts are final; make this launch's input
            finish_kernel<<<dim3(static_cast<unsigned>(t)), dim3(1024), hidden * sizeof(float), stream>>>(
                part, plan.parts, static_cast<int>(t), static_cast<int>(hidden), y, static_cast<std::uint16_t*>(x), eps,
                nullptr, nullptr, 0);
            check_launch("small-M stack finish launch");
        }
        p.layers = static_cast<int>(n);
        for (std::size_t i = 0; i < n; ++i) {
            p.w_gu[i] = reinterpret_cast<const signed char*>(w_gu[l0 + i]);
            p.s_gu[i] = s_gu[l0 + i];
            p.w_d[i] = reinterpret_cast<const signed char*>(w_d[l0 + i]);
            p.s_d[i] = s_d[l0 + i];
        }
        void* args[] = {&p};
        if (hipLaunchCooperativeKernel(reinterpret_cast<const void*>(stack_kernel), dim3(static_cast<unsigned>(plan.blocks)),
                                       dim3(kThreads), args, static_cast<unsigned>(lds), stream) != hipSuccess)
            throw LaunchError("small-M stack: cooperative launch failed");
    }
    return true;
}

} // namespace sepal::hip
