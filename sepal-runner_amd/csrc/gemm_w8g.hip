// gpu-w8g on gfx950: Y = epilogue(X * dequant(W)^T) with W int8 + one float32 scale per (row, 128 values of k).
//
// The reference multiplies fp32 X by the dequantised float32 weights in one fmaf chain per output
// (runner/cuda/src/gemm_simt_kernels.cu:71-240). Here the contraction runs on MFMA: the weight bytes are widened to the
// MFMA input type exactly (int8 has at most 8 significant bits, bf16 and binary16 hold it), X is bf16 or binary16, each
// product is exact in the float32 accumulator, and the per-group scales are applied outside the MFMA by the group
// identity Y = sum_g s_g * (sum_{k in g} x_k q_k) (proofs/GpuTrack/GpuTrack/GroupQuant.lean:38-50). To keep one set of
// accumulators, the scales are folded in Horner form: U_0 = P_0, U_g = U_{g-1} * (e_{g-1} / e_g) + P_g, Y = U_last *
// e_last, where P_g is the MFMA partial of group g accumulated straight into U and e_g is the group's scale (a zero
// scale keeps the previous one: its group's bytes are all zero). Results match the fmaf chain within float32 rounding
// of a different summation order, not bit for bit.
//
// Two paths:
//   large M: 256 x BN tiles (BN 128 or 256), 4 or 8 waves of 128 x 64 outputs (4 x 2 blocks of 32 x 32, MFMA
//            32x32x16), K in steps of BK through a double-buffered LDS tile; the weights are widened once per tile
//            when staged; 1-D grid with an XCD-aware tile order (a block's id modulo 8 is its XCD; consecutive logical
//            tiles are kept on one XCD so they share its L2).
//   small M: the weights are streamed once (HBM-bound): a block of 4 waves owns 64 weight rows and a range of K;
//            X (T <= 64 rows) is staged in LDS; MFMA 16x16x32; when K is split the float32 partials go to the
//            library workspace and the last block to arrive sums them in split order and applies the epilogue.
#include "common.hpp"
#include "gemm_kernels.hpp"

namespace sepal::hip {
namespace w8g {

// ---- shared helpers --------------------------------------------------------------------------------------------------

// Sixteen int8 weights (a 16-byte chunk) widened to the MFMA type: 8 dwords (16 elements) in k order.
template <int XT>
__device__ __forceinline__ void widen16(const u32x4 v, unsigned (&o)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (XT == SEPAL_HIP_BF16) s8x4_to_bf16x4(v[i], o[2 * i], o[2 * i + 1]);
        else s8x4_to_f16x4(v[i], o[2 * i], o[2 * i + 1]);
    }
}

template <int XT>
__device__ __forceinline__ f32x16 mfma32(const u32x4 a, const u32x4 b, f32x16 c) {
    if constexpr (XT == SEPAL_HIP_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <int XT>
__device__ __forceinline__ f32x4 mfma16(const u32x4 a, const u32x4 b, f32x4 c) {
    if constexpr (XT == SEPAL_HIP_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Effective scale of a group: a zero (or negative/NaN) scale marks an all-zero group and keeps the previous one.
__device__ __forceinline__ float next_scale(float s, float prev) { return s > 0.0f ? s : prev; }

// Epilogue of one output element (row, col) of the plain multiply.
template <int EP>
__device__ __forceinline__ void put_plain(float* y, std::size_t idx, float v) {
    if constexpr (EP == SEPAL_HIP_ADD) y[idx] = __fadd_rn(y[idx], v);
    else y[idx] = v;
}

// ---- large-M path ----------------------------------------------------------------------------------------------------

struct BigParams {
    const unsigned short* x;   // [T, ld_x] bf16 / binary16 bits
    std::size_t ld_x;
    const signed char* w;      // [N, ld_w]
    std::size_t ld_w;
    const float* s;            // [N, ld_s]
    std::size_t ld_s;
    void* y;
    std::size_t ld_y;
    int t, n, k;
    int tiles_m, tiles_n;
};

// Logical tile of block `bid` (XCD-aware: the hardware places block b on XCD b % 8).
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int total = tiles_m * tiles_n;
    const int q = total / 8, r = total % 8;
    const int xcd = bid % 8, idx = bid / 8;
    const int id = xcd * q + min(xcd, r) + idx;
    constexpr int GM = 4;  // M tiles per group: a group sweeps N with the same few X row panels
    const int per_group = GM * tiles_n;
    const int group = id / per_group, first_m = group * GM;
    const int gm = min(tiles_m - first_m, GM);
    const int in_group = id % per_group;
    tm = first_m + in_group % gm;
    tn = in_group / gm;
}

// LDS tiles hold rows of BK 16-bit elements in 16-byte chunks; chunk c of row r is stored at chunk c ^ swz(r).
template <int BK>
__device__ __forceinline__ int swz(int r) {
    constexpr int CPR = BK / 8;
    return CPR == 8 ? (r & 7) : ((r >> 1) & (CPR - 1));
}

template <int XT, int EP, int YT, int WN, int BK>
__global__ void __launch_bounds__(128 * WN) gemm_big(const BigParams p) {
    constexpr int NT = 128 * WN;        // threads (2 waves along M, WN along N)
    constexpr int BM = 256, BN = 64 * WN;
    constexpr int CPR = BK / 8;         // 16-byte chunks per LDS row
    constexpr int XCH = BM * CPR / NT;  // X chunks per thread per stage
    constexpr int WCH = BN * (BK / 16) / NT;  // 16-byte weight chunks per thread per stage
    constexpr int GPS = 128 / BK;       // K steps per scale group
    static_assert(XCH >= 1 && WCH >= 1 && GPS >= 1, "tile");

    __shared__ __align__(16) u32x4 lds_x[2][BM * CPR];
    __shared__ __align__(16) u32x4 lds_w[2][BN * CPR];

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int wm = wave % 2, wn = wave / 2;
    int tm, tn;
    tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    // global -> register staging
    u32x4 xr[XCH], wr[WCH];
    const auto gload = [&](int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int e = 0; e < XCH; ++e) {
            const int id = tid + e * NT, row = id / CPR, c = id % CPR;
            const int m = m0 + row;
            if (m < p.t) xr[e] = *reinterpret_cast<const u32x4*>(p.x + static_cast<std::size_t>(m) * p.ld_x + k0 + 8 * c);
            else xr[e] = u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int e = 0; e < WCH; ++e) {
            const int id = tid + e * NT, row = id / (BK / 16), c = id % (BK / 16);
            const int nn = n0 + row;
            if (nn < p.n) wr[e] = *reinterpret_cast<const u32x4*>(p.w + static_cast<std::size_t>(nn) * p.ld_w + k0 + 16 * c);
            else wr[e] = u32x4{0u, 0u, 0u, 0u};
        }
    };
    const auto lstore = [&](int buf) {
#pragma unroll
        for (int e = 0; e < XCH; ++e) {
            const int id = tid + e * NT, row = id / CPR, c = id % CPR;
            lds_x[buf][row * CPR + (c ^ swz<BK>(row))] = xr[e];
        }
#pragma unroll
        for (int e = 0; e < WCH; ++e) {
            const int id = tid + e * NT, row = id / (BK / 16), c = id % (BK / 16);
            unsigned o[8];
            widen16<XT>(wr[e], o);
            const int c0 = 2 * c, c1 = 2 * c + 1;
            lds_w[buf][row * CPR + (c0 ^ swz<BK>(row))] = u32x4{o[0], o[1], o[2], o[3]};
            lds_w[buf][row * CPR + (c1 ^ swz<BK>(row))] = u32x4{o[4], o[5], o[6], o[7]};
        }
    };

    // This lane's output columns: block nb = 0 (gate half for SwiGLU) and 1 (the matching up half).
    const int ib = wn / 2, hh = wn % 2;
    const int colrel[2] = {128 * ib + 32 * hh + lane % 32, 128 * ib + 64 + 32 * hh + lane % 32};
    int col[2];
    const float* srow[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        col[j] = n0 + colrel[j];
        srow[j] = col[j] < p.n ? p.s + static_cast<std::size_t>(col[j]) * p.ld_s : nullptr;
    }
    const auto scale_at = [&](int j, int g) -> float { return srow[j] != nullptr ? srow[j][g] : 1.0f; };

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    float e[2], snext[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        e[j] = next_scale(scale_at(j, 0), 1.0f);
        snext[j] = p.k > 128 ? scale_at(j, 1) : 1.0f;
    }

    const int KT = p.k / BK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < KT) gload(kt + 1);
        if (kt > 0 && kt % GPS == 0) {
            const int g = kt / GPS;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float en = next_scale(snext[j], e[j]);
                const float ratio = e[j] / en;
                e[j] = en;
                snext[j] = (g + 1) * 128 < p.k ? scale_at(j, g + 1) : 1.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = __fmul_rn(acc[i][j][r], ratio);
            }
        }
        const u32x4* tx = lds_x[buf];
        const u32x4* tw = lds_w[buf];
#pragma unroll
        for (int st = 0; st < BK / 16; ++st) {
            const int c = 2 * st + lane / 32;
            u32x4 a[4], b[2];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = wm * 128 + i * 32 + lane % 32;
                a[i] = tx[row * CPR + (c ^ swz<BK>(row))];
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int row = colrel[j];
                b[j] = tw[row * CPR + (c ^ swz<BK>(row))];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma32<XT>(a[i], b[j], acc[i][j]);
        }
        if (kt + 1 < KT) lstore(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue ----
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + wm * 128 + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
            if (row >= p.t) continue;
            const float v0 = __fmul_rn(acc[i][0][r], e[0]), v1 = __fmul_rn(acc[i][1][r], e[1]);
            if constexpr (EP == SEPAL_HIP_SWIGLU) {
                const int f = n0 / 2 + 64 * ib + 32 * hh + lane % 32;
                if (2 * f < p.n) store_out<YT>(p.y, static_cast<std::size_t>(row) * p.ld_y + f, swiglu_libm(v0, v1));
            } else {
                float* y = static_cast<float*>(p.y);
                if (col[0] < p.n) put_plain<EP>(y, static_cast<std::size_t>(row) * p.ld_y + col[0], v0);
                if (col[1] < p.n) put_plain<EP>(y, static_cast<std::size_t>(row) * p.ld_y + col[1], v1);
            }
        }
    }
}

// ---- small-M path ----------------------------------------------------------------------------------------------------

struct SmallParams {
    const unsigned short* x;   // [T, ld_x] bf16 / binary16 bits
    std::size_t ld_x;
    const signed char* w;
    std::size_t ld_w;
    const float* s;
    std::size_t ld_s;
    void* y;
    std::size_t ld_y;
    int t, n, k;
    int splits;                // K splits (1: no workspace)
    int groups_per_split;      // scale groups per split
    float* partial;            // [splits][T][n_cols_padded] when splits > 1
    unsigned* counters;        // one per column block when splits > 1
    int col_blocks;
};

// Column of wave-slot `slot` (0..63) of column block `cb`: SwiGLU blocks take 32 gate and the matching 32 up columns.
template <int EP>
__device__ __forceinline__ int small_col(int cb, int slot) {
    if constexpr (EP == SEPAL_HIP_SWIGLU) {
        const int b = cb / 2, h = cb % 2;
        return slot < 32 ? 128 * b + 32 * h + slot : 128 * b + 64 + 32 * h + (slot - 32);
    } else {
        return 64 * cb + slot;
    }
}

// MT: 16-row blocks of X (T <= 16 MT). KR_MAX: the largest K range of one split (LDS holds X[T][KR]).
template <int XT, int EP, int YT, int MT>
__global__ void __launch_bounds__(256) gemm_small(const SmallParams p) {
    constexpr int KR_MAX = small_kr_max(MT);
    __shared__ __align__(16) unsigned short lds_x[16 * MT * KR_MAX];  // X slice, row stride KR_MAX
    __shared__ float red[4][16 * MT][16];                                // SwiGLU / reduction exchange

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int cb = blockIdx.x % p.col_blocks, ks = blockIdx.x / p.col_blocks;
    const int g0 = ks * p.groups_per_split;
    const int g1 = min(g0 + p.groups_per_split, p.k / 128);
    const int kbeg = g0 * 128, klen = (g1 - g0) * 128;

    // stage X[0..T)[kbeg, kbeg + klen) (16-byte chunks, zero rows beyond T)
    {
        const int cpr = klen / 8;
        for (int id = tid; id < 16 * MT * cpr; id += 256) {
            const int r = id / cpr, c = id % cpr;
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (r < p.t) v = *reinterpret_cast<const u32x4*>(p.x + static_cast<std::size_t>(r) * p.ld_x + kbeg + 8 * c);
            *reinterpret_cast<u32x4*>(&lds_x[r * KR_MAX + 8 * c]) = v;
        }
    }
    __syncthreads();

    // this wave: 16 weight rows; lane reads row (lane % 16), 16 bytes at k offset 16 * (lane / 16) of every 64-k chunk
    const int slot0 = wave * 16;
    const int colw = small_col<EP>(cb, slot0 + lane % 16);
    const bool col_ok = colw < p.n;
    const signed char* wrow = p.w + static_cast<std::size_t>(col_ok ? colw : 0) * p.ld_w;
    const float* srow = p.s + static_cast<std::size_t>(col_ok ? colw : 0) * p.ld_s;

    f32x4 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float e = 1.0f;

    constexpr int PF = 4;  // groups of weight loads in flight
    u32x4 wbuf[PF][2];
    const auto wload = [&](int g, u32x4 (&dst)[2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = g * 128 + 64 * h + 16 * (lane / 16);
            dst[h] = col_ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + k)) : u32x4{0u, 0u, 0u, 0u};
        }
    };
#pragma unroll
    for (int i = 0; i < PF; ++i)
        if (g0 + i < g1) wload(g0 + i, wbuf[i]);

    for (int gb = g0; gb < g1; gb += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int g = gb + u;
            if (g >= g1) break;
            const float sg = col_ok ? srow[g] : 1.0f;
            const float en = next_scale(sg, e);
            if (g > g0) {
                const float ratio = e / en;
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][r] = __fmul_rn(acc[i][r], ratio);
            }
            e = en;
            u32x4 cur[2] = {wbuf[u][0], wbuf[u][1]};
            if (g + PF < g1) wload(g + PF, wbuf[u]);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                unsigned o[8];
                widen16<XT>(cur[h], o);
                const u32x4 b0 = u32x4{o[0], o[1], o[2], o[3]}, b1 = u32x4{o[4], o[5], o[6], o[7]};
                const int kl = (g - g0) * 128 + 64 * h + 16 * (lane / 16);
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    const unsigned short* xr = &lds_x[(16 * i + lane % 16) * KR_MAX + kl];
                    const u32x4 a0 = *reinterpret_cast<const u32x4*>(xr);
                    const u32x4 a1 = *reinterpret_cast<const u32x4*>(xr + 8);
                    acc[i] = mfma16<XT>(a0, b0, acc[i]);
                    acc[i] = mfma16<XT>(a1, b1, acc[i]);
                }
            }
        }
    }
    // acc[i][r]: row 16 i + 4 (lane / 16) + r, column slot0 + lane % 16 of the block
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][r] = __fmul_rn(acc[i][r], e);

    const int ncols_pad = p.col_blocks * 64;
    if (p.splits > 1) {
        // write this split's partial, then the last block of the column block reduces in split order
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * i + 4 * (lane / 16) + r;
                p.partial[(static_cast<std::size_t>(ks) * 16 * MT + row) * ncols_pad + cb * 64 + slot0 + lane % 16] = acc[i][r];
            }
        __threadfence();
        __syncthreads();
        __shared__ unsigned last;
        if (tid == 0) {
            const unsigned prev = atomicAdd(&p.counters[cb], 1u);
            last = prev == static_cast<unsigned>(p.splits - 1) ? 1u : 0u;
        }
        __syncthreads();
        if (last == 0u) return;
        __threadfence();
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * i + 4 * (lane / 16) + r;
                float v = 0.0f;
                for (int s = 0; s < p.splits; ++s) {
                    const float* src = p.partial + (static_cast<std::size_t>(s) * 16 * MT + row) * ncols_pad + cb * 64 + slot0 + lane % 16;
                    v = s == 0 ? __builtin_nontemporal_load(src) : __fadd_rn(v, __builtin_nontemporal_load(src));
                }
                acc[i][r] = v;
            }
        if (tid == 0) p.counters[cb] = 0u;
    }

    if constexpr (EP == SEPAL_HIP_SWIGLU) {
        // waves 2, 3 hold the up columns of waves 0, 1
        if (wave >= 2) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) red[wave - 2][16 * i + 4 * (lane / 16) + r][lane % 16] = acc[i][r];
        }
        __syncthreads();
        if (wave < 2) {
            const int f = (cb / 2) * 64 + (cb % 2) * 32 + wave * 16 + lane % 16;
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = 16 * i + 4 * (lane / 16) + r;
                    if (row < p.t && 2 * f < p.n)
                        store_out<YT>(p.y, static_cast<std::size_t>(row) * p.ld_y + f, swiglu_libm(acc[i][r], red[wave][row][lane % 16]));
                }
        }
    } else {
        float* y = static_cast<float*>(p.y);
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * i + 4 * (lane / 16) + r;
                if (row < p.t && col_ok) put_plain<EP>(y, static_cast<std::size_t>(row) * p.ld_y + colw, acc[i][r]);
            }
    }
}

// ---- launch ----------------------------------------------------------------------------------------------------------

template <int XT, int EP, int YT>
void launch_big(const GemmArgs& a, hipStream_t stream) {
    BigParams p{static_cast<const unsigned short*>(a.x), a.ld_x, reinterpret_cast<const signed char*>(a.w), a.ld_w, a.s, a.ld_s,
                a.y, a.ld_y, static_cast<int>(a.t), static_cast<int>(a.n), static_cast<int>(a.k), 0, 0};
    // 256 x 256 tiles when there are enough of them to fill the chip twice, else 256 x 128
    const int tiles_m = static_cast<int>((a.t + 255) / 256);
    const int tn256 = static_cast<int>((a.n + 255) / 256);
    const bool wide = static_cast<long>(tiles_m) * tn256 >= 2 * 256 && (EP != SEPAL_HIP_SWIGLU || a.n % 256 == 0);
    p.tiles_m = tiles_m;
    if (wide) {
        p.tiles_n = tn256;
        gemm_big<XT, EP, YT, 4, 64><<<dim3(tiles_m * p.tiles_n), dim3(512), 0, stream>>>(p);
    } else {
        p.tiles_n = static_cast<int>((a.n + 127) / 128);
        gemm_big<XT, EP, YT, 2, 32><<<dim3(tiles_m * p.tiles_n), dim3(256), 0, stream>>>(p);
    }
    check_launch("gemm_w8g large-M kernel launch");
}

template <int XT, int EP, int YT, int MT>
void launch_small_mt(const GemmArgs& a, hipStream_t stream) {
    SmallParams p{};
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
    p.col_blocks = static_cast<int>((a.n + 63) / 64);
    const int groups = p.k / 128;
    // enough blocks to keep every CU streaming (about 2 per CU), one split's X slice within the LDS tile
    const int max_gps = small_kr_max(MT) / 128;
    int splits = (2 * 256 + p.col_blocks - 1) / p.col_blocks;
    splits = max(splits, (groups + max_gps - 1) / max_gps);
    splits = min(splits, groups);
    if (a.force_splits > 0) splits = min(a.force_splits, groups);
    p.groups_per_split = (groups + splits - 1) / splits;
    splits = (groups + p.groups_per_split - 1) / p.groups_per_split;
    require(p.groups_per_split <= max_gps, "gemm_w8g small-M: split too long for LDS");
    p.splits = splits;
    if (splits > 1) {
        const std::size_t part = static_cast<std::size_t>(splits) * 16 * MT * p.col_blocks * 64 * sizeof(float);
        require(static_cast<std::size_t>(p.col_blocks) * sizeof(unsigned) <= kCounterBytes && part <= kPartialBytes,
                "small-M multiply: workspace zone too small for this shape");
        char* ws = static_cast<char*>(workspace(kScratchOffset, stream));
        p.counters = reinterpret_cast<unsigned*>(ws);
        p.partial = reinterpret_cast<float*>(ws + kCounterBytes);
    }
    gemm_small<XT, EP, YT, MT><<<dim3(p.col_blocks * splits), dim3(256), 0, stream>>>(p);
    check_launch("gemm_w8g small-M kernel launch");
}

template <int XT, int EP, int YT>
void launch_small(const GemmArgs& a, hipStream_t stream) {
    const std::size_t mt = (a.t + 15) / 16;
    switch (mt) {
    case 1: launch_small_mt<XT, EP, YT, 1>(a, stream); break;
    case 2: launch_small_mt<XT, EP, YT, 2>(a, stream); break;
    case 3: launch_small_mt<XT, EP, YT, 3>(a, stream); break;
    default: launch_small_mt<XT, EP, YT, 4>(a, stream); break;
    }
}

template <int XT, int EP, int YT>
void dispatch_path(const GemmArgs& a, hipStream_t stream) {
    const bool small = a.config == 1 || (a.config < 0 && a.t <= kSmallM);
    if (small) launch_small<XT, EP, YT>(a, stream);
    else launch_big<XT, EP, YT>(a, stream);
}

template <int XT>
void dispatch_ep(const GemmArgs& a, hipStream_t stream) {
    switch (a.epilogue) {
    case SEPAL_HIP_STORE: dispatch_path<XT, SEPAL_HIP_STORE, SEPAL_HIP_F32>(a, stream); break;
    case SEPAL_HIP_ADD: dispatch_path<XT, SEPAL_HIP_ADD, SEPAL_HIP_F32>(a, stream); break;
    default:
        switch (a.y_type) {
        case SEPAL_HIP_F32: dispatch_path<XT, SEPAL_HIP_SWIGLU, SEPAL_HIP_F32>(a, stream); break;
        case SEPAL_HIP_BF16: dispatch_path<XT, SEPAL_HIP_SWIGLU, SEPAL_HIP_BF16>(a, stream); break;
        default: dispatch_path<XT, SEPAL_HIP_SWIGLU, SEPAL_HIP_F16>(a, stream); break;
        }
    }
}

} // namespace w8g

void launch_gemm_w8g(const GemmArgs& a, hipStream_t stream) {
    if (a.x_type == SEPAL_HIP_BF16) w8g::dispatch_ep<SEPAL_HIP_BF16>(a, stream);
    else w8g::dispatch_ep<SEPAL_HIP_F16>(a, stream);
}

} // namespace sepal::hip
