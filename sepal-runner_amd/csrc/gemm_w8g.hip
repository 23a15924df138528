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
// Paths:
//   large M: waves of 128 x 64 outputs (4 x 2 blocks of 32 x 32, MFMA 32x32x16; 64 x 64 in the half tiles); 1-D grid
//            with an XCD-aware tile order (a block's id modulo 8 is its XCD; consecutive logical tiles are kept on one
//            XCD so they share its L2). Grids of at least two rounds of 256 x 256 tiles: the weights are widened once
//            per call into an image of the W stages (widen_image_kernel, one streaming pass), which gemm_pp (two wave
//            groups in alternation) and the half tiles of gemm_big3 load straight into LDS. Otherwise the weights are
//            widened per tile by the waves when staged into LDS. gemm_big3:
//            256 x 256 tiles (128 x 256 halves for a launch's last partial round; for grids of fewer than 512 large
//            tiles, blocks of 64, 128 or 256 rows and, by default, K split over blocks with the partials added by the
//            last block of a tile or by planes_sum_kernel, and the leading whole 256-row tiles run apart from the rows
//            after them, by plan_small_grid), K in steps of 64, X straight from global memory into LDS. gemm_big2 (when an offset does not fit 32 bits, or a
//            SwiGLU N is not a multiple of 256): 256 x 128 or 256 x 256 tiles, K in steps of 32.
//   small M: at T <= 16 the M <= 16 stack's pass kernels (stack_small.hip) where the shape fits them; else, at
//            T <= 32 with N < 8192, stream.hip (the weights streamed once, HBM-bound); else the large-M plan.
#include <algorithm>
#include <atomic>

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

// Items [id0, total) of the weight image, every id_stride-th (the layout at widen_image_kernel): item id widens one
// 16-byte chunk (16 values of one substep) of one weight row into its two 16-byte slots of the image, exactly, to
// binary16 (f16) or bf16. Eight consecutive items are the eight chunks of 128 bytes of one row (two 64-value steps),
// so a wave reads 8 rows x 128 contiguous bytes and writes 128-byte runs.
__device__ __forceinline__ void widen_range(const signed char* __restrict__ w, std::size_t ld_w, int n, int wsteps, int tiles_n,
                                            unsigned char* __restrict__ img, bool f16, std::size_t id0, std::size_t id_stride) {
    const int pairs = wsteps / 2;
    const std::size_t total = static_cast<std::size_t>(tiles_n) * pairs * 256 * 8;
    for (std::size_t id = id0; id < total; id += id_stride) {
        const int j = static_cast<int>(id % 8), c = static_cast<int>((id / 8) % 32), nb = static_cast<int>((id / 256) % 8);
        const int kp = static_cast<int>((id / 2048) % pairs), tn = static_cast<int>(id / 2048 / pairs);
        const int row = tn * 256 + nb * 32 + c;
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (row < n) v = *reinterpret_cast<const u32x4*>(w + static_cast<std::size_t>(row) * ld_w + 128 * kp + 16 * j);
        const int h = j / 4, st = j % 4;
        unsigned char* const stage = img + (static_cast<std::size_t>(tn) * wsteps + 2 * kp + h) * 32768;
        unsigned o[8];
        if (f16) widen16<SEPAL_HIP_F16>(v, o);
        else widen16<SEPAL_HIP_BF16>(v, o);
        *reinterpret_cast<u32x4*>(stage + (nb * 4 + st) * 1024 + c * 16) = u32x4{o[0], o[1], o[2], o[3]};
        *reinterpret_cast<u32x4*>(stage + (nb * 4 + st) * 1024 + (c + 32) * 16) = u32x4{o[4], o[5], o[6], o[7]};
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

// The SwiGLU output f of `row` (the output's row stride ld_y values) as YT, or, for kYPairs, as its bf16 hi + lo
// pair in the hi + lo row layout the 64-wide-step kernel reads (row stride 2 ld_y; value f at 128 (f / 64) + f % 64,
// its lo 64 values on): the rounding of the split pass on the float32 value, so the down multiply's bits are those
// of float32 H split by that pass.
template <int YT>
__device__ __forceinline__ void store_h(void* y, std::size_t row, std::size_t ld_y, int f, float v) {
    if constexpr (YT == kYPairs) {
        unsigned short* const d = static_cast<unsigned short*>(y) + row * 2 * ld_y + 128 * (f / 64) + f % 64;
        const unsigned short h = f32_to_bf16_bits(v);
        d[0] = h;
        d[64] = f32_to_bf16_bits(__fsub_rn(v, bf16_bits_to_f32(h)));
    } else {
        store_out<YT>(y, row * ld_y + f, v);
    }
}

// Epilogue of one output element (row, col) of the plain multiply: float32 Store / Add, or a binary16 Store (the
// float32 value rounded to nearest even, as a separate conversion would).
template <int EP, int YT>
__device__ __forceinline__ void put_plain(void* y, std::size_t idx, float v) {
    if constexpr (YT != SEPAL_HIP_F32) {
        static_assert(EP == SEPAL_HIP_STORE, "16-bit outputs of the plain multiply are Store only");
        store_out<YT>(y, idx, v);
    } else if constexpr (EP == SEPAL_HIP_ADD) {
        static_cast<float*>(y)[idx] = __fadd_rn(static_cast<float*>(y)[idx], v);
    } else {
        static_cast<float*>(y)[idx] = v;
    }
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
    std::size_t x_bytes, w_bytes;  // extents of X and W (buffer range checks of gemm_big3)
    int id0 = 0, count = 0;        // gemm_big3: the logical 256 x 256 tiles [id0, id0 + count) of this launch
    // gemm_big3 split-K: each block tile (BM3 x 256) is computed by `splits` blocks over consecutive ranges of whole
    // groups; each writes its float32 partial to `part` and counts in on counters[tile]; the last to arrive adds the
    // partials in split order and runs the epilogue
    int splits = 1;
    float* part = nullptr;
    unsigned* counters = nullptr;
    // split-K launches run the live block tiles sub0 .. sub0 + nsub - 1 of the dense order: block tile s at rows
    // (s mod sub_m) BM3 and columns (s / sub_m) 256, sub_m = ceil(T / BM3)
    int dense = 0, sub_m = 0, sub0 = 0, nsub = 0;
    // split-K into planes: instead of the hand-off, split s writes its float32 partial (the same values) row-major to
    // part + s * t * n (row stride n), and planes_sum_kernel adds the planes in split order and runs the epilogue
    int planes = 0;
    // gemm_pp: the widened W stage of 256-column tile tn and weight step ks (64 values of k) is the 32 KB at wimg +
    // (tn * wsteps + ks) * 32768, in the LDS order the fragment reads use
    const unsigned char* wimg = nullptr;
    std::size_t wimg_bytes = 0;
    int wsteps = 0;
    // a second weight image widened by extra blocks of the halves launch (the blocks past the halves), for the next
    // multiply of a stack: its weights, shape and destination
    const signed char* jw = nullptr;
    std::size_t j_ld = 0;
    int j_n = 0, j_wsteps = 0, j_tiles_n = 0, j_f16 = 0, j_blocks = 0;
    unsigned char* j_img = nullptr;
};

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

// Logical id of block `bid` among `total` (XCD-aware: the hardware places block b on XCD b % 8, and each XCD takes a
// contiguous range of ids, so that consecutive tiles share its L2).
__device__ __forceinline__ int xcd_id(int bid, int total) {
    const int q = total / 8, r = total % 8;
    const int xcd = bid % 8, idx = bid / 8;
    return xcd * q + min(xcd, r) + idx;
}

__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
    tile_from_id(xcd_id(bid, tiles_m * tiles_n), tiles_m, tiles_n, tm, tn);
}

// ---- large-M kernel for small grids: fragment-order LDS, 32-wide k steps (gemm_big2) ---------------------------------
//
// LDS holds every MFMA operand fragment in the order a wave reads it: fragment (block b, substep st) is 64 lanes x 16
// bytes, lane l at byte 16 l, so an operand read is one contiguous kilobyte (no bank conflicts, one address per lane
// for the whole kernel). Each lane loads into registers the 16 bytes of X it will later read (row mb*32 + l%32, k
// 16st + 8(l/32)) and writes them to its slot; a W fragment is filled by the wave that widens the weight bytes (row
// nb*32 + l%32, k 16st .. 16st + 15 -> lanes l%32 and 32 + l%32). K runs in steps of 32 through two LDS stages; the
// loads of step kt + 3 are issued while step kt is multiplied (four rotating register sets), and one barrier per step
// publishes step kt + 1. Each lane's two column scales come with the group's loads.
namespace v2 {

constexpr int BM = 256, BK = 32, STAGES = 2;

typedef __attribute__((address_space(3))) unsigned char lds_byte;
typedef const __attribute__((address_space(1))) void global_void;

// s_waitcnt with only the vector memory counter limited (gfx9 encoding: vmcnt[3:0] bits 3:0, vmcnt[5:4] bits 15:14;
// expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <int XT, int EP, int YT, int WN>
__global__ void __launch_bounds__(128 * WN) __attribute__((amdgpu_waves_per_eu(2))) gemm_big2(const BigParams p) {
    constexpr int NT = 128 * WN, NW = NT / 64;   // threads, waves (2 along M, WN along N; each 128 x 64 outputs)
    constexpr int BN = 64 * WN;
    constexpr int SPG = 128 / BK;                 // steps per scale group
    constexpr int XF = (BM / 32) * (BK / 16);     // X fragments per stage (16)
    constexpr int WF = (BN / 32) * (BK / 16);     // W fragments per stage (4 WN)
    constexpr int XFPW = XF / NW;                 // X fragments each wave loads per stage
    constexpr int XSTAGE = XF * 1024, WSTAGE = WF * 1024;
    static_assert(WF == 2 * NW, "one W chunk per thread per stage");
    extern __shared__ __align__(16) unsigned char smem[];
    lds_byte* lds = (lds_byte*)smem;  // generic -> LDS address space (a C cast is the one that may change it)
    lds_byte* xs_base = lds;                                 // [STAGES][XF][1 KB]
    lds_byte* ws_base = lds + STAGES * XSTAGE;                // [STAGES][WF][1 KB]

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int wm = wave % 2, wn = wave / 2;
    int tm, tn;
    tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int KT = p.k / BK;

    // ---- per-lane global sources (clamped: rows past T or N repeat the last row, never stored) ----
    const u32x4* xsrc[XFPW];
#pragma unroll
    for (int i = 0; i < XFPW; ++i) {
        const int f = wave * XFPW + i, mb = f / (BK / 16), st = f % (BK / 16);
        const int row = min(m0 + mb * 32 + lane % 32, p.t - 1);
        xsrc[i] = reinterpret_cast<const u32x4*>(p.x + static_cast<std::size_t>(row) * p.ld_x + 16 * st + 8 * (lane / 32));
    }
    const int wrow_n = min(n0 + 32 * wave + lane % 32, p.n - 1);
    const signed char* wsrc = p.w + static_cast<std::size_t>(wrow_n) * p.ld_w + 16 * (lane / 32);
    const int wfrag = wave * 2 + lane / 32;  // the W fragment this lane widens (n-block = wave, substep = lane / 32)

    // this lane's output columns: n-block j = 0 (gate half for SwiGLU) and 1 (the matching up half; gate and up
    // alternate every 64 columns)
    const int ib = wn / 2, hh = wn % 2;
    const int nbj[2] = {4 * ib + hh, 4 * ib + 2 + hh};
    int col[2];
    const float* ssrc[2];  // scale rows of the two columns
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        col[j] = n0 + 32 * nbj[j] + lane % 32;
        ssrc[j] = p.s + static_cast<std::size_t>(min(col[j], p.n - 1)) * p.ld_s;
    }

    // one step's operands, loaded into registers: the lane's X fragment chunks and W chunk
    struct Regs {
        u32x4 x[XFPW];
        u32x4 w;
    };
    float snext[2];  // the next group's scales, loaded ahead of its first step's operands
    const auto issue = [&](int kt, Regs& r) {
#pragma unroll
        for (int i = 0; i < XFPW; ++i) r.x[i] = xsrc[i][static_cast<std::size_t>(kt) * (BK * 2 / 16)];
        r.w = *reinterpret_cast<const u32x4*>(wsrc + static_cast<std::size_t>(kt) * BK);
    };
    const auto issue_scales = [&](int g) {
        snext[0] = ssrc[0][g];
        snext[1] = ssrc[1][g];
    };
    // the step's operands into its LDS stage, in fragment order, the weights widened exactly to the MFMA type
    const auto stage = [&](int kt, const Regs& r) {
        lds_byte* xd = xs_base + (kt % STAGES) * XSTAGE + 16 * lane;
#pragma unroll
        for (int i = 0; i < XFPW; ++i)
            *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(xd + (wave * XFPW + i) * 1024) = r.x[i];
        unsigned o[8];
        widen16<XT>(r.w, o);
        lds_byte* wd = ws_base + (kt % STAGES) * WSTAGE + wfrag * 1024 + 16 * (lane % 32);
        *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(wd) = u32x4{o[0], o[1], o[2], o[3]};
        *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(wd + 512) = u32x4{o[4], o[5], o[6], o[7]};
    };

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // ---- prologue: group 0's scales, steps 0, 1, 2 in flight; step 0 staged ----
    Regs r0, r1, r2, r3;
    issue_scales(0);
    issue(0, r0);
    issue(1, r1);
    issue(2, r2);
    stage(0, r0);
    __syncthreads();
    // the Horner state (the first step's factor multiplies zero accumulators)
    float e[2] = {1.0f, 1.0f}, emax[2] = {0.0f, 0.0f};

    // One step: issue step kt + 3's loads into the registers of step kt - 1 (the next group's scales first when
    // kt + 3 starts a group); at a group's first step the Horner rescale; the multiply of step kt; then stage step
    // kt + 1's operands (loaded two steps ago; the stage was last read by step kt - 1); one barrier. The load registers
    // rotate through four names, step s in R[s % 4], and the loop runs one group (four steps) per iteration, so the
    // rotation is a renaming and the group boundary is known at compile time. The body has no branches, so the
    // compiler's load counting stays exact: near the end the loads repeat the last step (clamped) and the extra stage
    // written at the last step lands in a buffer nothing reads again. At step 0 the rescale multiplies zero
    // accumulators.
    const int groups = KT / SPG;
    const auto step = [&](int kt, const Regs& r_next, Regs& r_free, auto first_t) {
        constexpr bool first = decltype(first_t)::value;
        if ((kt + 3) % SPG == 0) issue_scales(min((kt + 3) / SPG, groups - 1));
        issue(min(kt + 3, KT - 1), r_free);
        if constexpr (first) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float ratio = horner_step(snext[j], e[j], emax[j]);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i][j] = acc[i][j] * ratio;
            }
        }
        const lds_byte* xs = xs_base + (kt % STAGES) * XSTAGE + 16 * lane;
        const lds_byte* ws = ws_base + (kt % STAGES) * WSTAGE + 16 * lane;
#pragma unroll
        for (int st = 0; st < BK / 16; ++st) {
            u32x4 a[4], b[2];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                a[i] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(xs + ((wm * 4 + i) * (BK / 16) + st) * 1024);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(ws + (nbj[j] * (BK / 16) + st) * 1024);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma32<XT>(a[i], b[j], acc[i][j]);
        }
        // step kt + 1's operands into their stage after this step's fragment reads, so that the writes overlap the
        // MFMAs instead of delaying their operands
        stage(kt + 1, r_next);
        __syncthreads();
    };
    static_assert(SPG == 4, "four steps per group");
    for (int kt = 0; kt < KT; kt += 4) {
        step(kt, r1, r3, std::true_type{});        // R1 holds step kt+1, step kt+3 -> R3
        step(kt + 1, r2, r0, std::false_type{});   // R2 holds kt+2, kt+4 -> R0
        step(kt + 2, r3, r1, std::false_type{});   // R3 holds kt+3, kt+5 -> R1
        step(kt + 3, r0, r2, std::false_type{});   // R0 holds kt+4, kt+6 -> R2
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
                if (2 * f < p.n) store_out<YT>(p.y, static_cast<std::size_t>(row) * p.ld_y + f, swiglu_fast(v0, v1));
            } else {
                if (col[0] < p.n) put_plain<EP, YT>(p.y, static_cast<std::size_t>(row) * p.ld_y + col[0], v0);
                if (col[1] < p.n) put_plain<EP, YT>(p.y, static_cast<std::size_t>(row) * p.ld_y + col[1], v1);
            }
        }
    }
}


// ---- large-M kernel, 64-wide k steps, X straight into LDS -----------------------------------------------------------
//
// The tile, waves and Horner scaling of gemm_big2, with K in steps of 64.
//   X: buffer_load ... lds (16 bytes a lane) writes the step's 256 x 64 tile straight into LDS, row-major with 128-byte
//      rows, chunk c of row r at slot c ^ ((r / 2) & 7): each 8 lanes of a load instruction read one whole cache line,
//      and every 16 lanes of an MFMA fragment read (16 rows, one chunk) cover the 16 bank groups. Three X stages; the
//      loads of step kt + 2 are issued while step kt is multiplied.
//   W: the int8 bytes come to registers two steps ahead (16 rows x 64 bytes per instruction) and are widened into a
//      fragment-ordered stage (lane L's 16 bytes at slot L ^ ((2 st + L / 32) & 7), st the 16-wide substep). Two
//      stages.
// The five stages are separate LDS arrays and the loop is unrolled over six steps, so that the compiler sees which
// array each direct load writes: a fragment read waits only for loads into the array it reads. Each step publishes
// its successor with a bare s_barrier after an explicit wait, since a workgroup release fence waits for every direct
// load in flight, including the ones two steps ahead.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));  // vmcnt(N) lgkmcnt(0)
}

// The epilogue of a 256-column tile of the large-M kernels: wave `wave` holds MB x 2 blocks of 32 x 32 outputs (rows
// m0 + 32 MB wm + 32 i.., columns n0 + 32 nbj[q]..), its Horner state e, and applies the last scale and the epilogue.
// OVERLAP (the persistent gemm_pp, whose next tile's first loads are in flight): a whole tile's values are computed
// first, in place, then the wave waits for its loads and issues the stores, which the next tile does not wait for;
// an edge tile waits for the loads, stores, and waits for its stores. Plain Add epilogues read y, so they keep the
// interleaved form.
template <int EP, int YT, int MB, bool OVERLAP = false>
__device__ __forceinline__ void tile_epilogue(const BigParams& p, f32x16 (&acc)[MB][2], const float (&e)[2], int m0, int n0,
                                              int wave, int lane) {
    constexpr int BM3 = 64 * MB, BN = 256;
    const int wm = wave % 2, wn = wave / 2, ib = wn / 2, hh = wn % 2;
    const int col[2] = {n0 + 32 * (4 * ib + hh) + lane % 32, n0 + 32 * (4 * ib + 2 + hh) + lane % 32};
    // A whole tile needs no bounds checks: the row and the wave's column base are wave-uniform (scalar registers) and
    // the lane adds a 32-bit offset, so a store costs no vector address arithmetic.
    if constexpr (OVERLAP && EP != SEPAL_HIP_ADD) {
        if (m0 + BM3 <= p.t && n0 + BN <= p.n) {
            constexpr unsigned ES = YT == SEPAL_HIP_F32 ? 4 : 2;
#pragma unroll
            for (int i = 0; i < MB; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float v0 = __fmul_rn(acc[i][0][r], e[0]), v1 = __fmul_rn(acc[i][1][r], e[1]);
                    if constexpr (EP == SEPAL_HIP_SWIGLU) {
                        acc[i][0][r] = swiglu_fast(v0, v1);
                    } else {
                        acc[i][0][r] = v0;
                        acc[i][1][r] = v1;
                    }
                }
            // the next tile's first loads (issued before this epilogue) are complete before the stores are queued
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("" ::: "memory");
            wait_vmcnt<0>();
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            const int wu = __builtin_amdgcn_readfirstlane(wave);
            const int wmu = wu % 2, ibu = (wu / 2) / 2, hhu = (wu / 2) % 2;
            const unsigned voff = (4u * static_cast<unsigned>(lane / 32) * static_cast<unsigned>(p.ld_y) + lane % 32) * ES;
            char* const yb = static_cast<char*>(p.y);
#pragma unroll
            for (int i = 0; i < MB; ++i) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const std::size_t row = static_cast<std::size_t>(m0 + wmu * 32 * MB + i * 32 + 8 * (r / 4) + (r % 4));
                    if constexpr (EP == SEPAL_HIP_SWIGLU && YT == kYPairs) {
                        store_h<YT>(p.y, row + 4 * (lane / 32), p.ld_y, n0 / 2 + 64 * ibu + 32 * hhu + lane % 32, acc[i][0][r]);
                    } else if constexpr (EP == SEPAL_HIP_SWIGLU) {
                        char* const rp = yb + (row * p.ld_y + n0 / 2 + 64 * ibu + 32 * hhu) * ES;
                        store_out<YT>(rp + voff, 0, acc[i][0][r]);
                    } else {
                        char* const rp0 = yb + (row * p.ld_y + n0 + 32 * (4 * ibu + hhu)) * ES;
                        char* const rp1 = yb + (row * p.ld_y + n0 + 32 * (4 * ibu + 2 + hhu)) * ES;
                        put_plain<EP, YT>(rp0 + voff, 0, acc[i][0][r]);
                        put_plain<EP, YT>(rp1 + voff, 0, acc[i][1][r]);
                    }
                }
            }
            return;
        }
    }
    if constexpr (OVERLAP) wait_vmcnt<0>();
    if (m0 + BM3 <= p.t && n0 + BN <= p.n) {
        constexpr unsigned ES = YT == SEPAL_HIP_F32 ? 4 : 2;
        const int wu = __builtin_amdgcn_readfirstlane(wave);
        const int wmu = wu % 2, ibu = (wu / 2) / 2, hhu = (wu / 2) % 2;
        const unsigned voff = (4u * static_cast<unsigned>(lane / 32) * static_cast<unsigned>(p.ld_y) + lane % 32) * ES;
        char* const yb = static_cast<char*>(p.y);
#pragma unroll
        for (int i = 0; i < MB; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const std::size_t row = static_cast<std::size_t>(m0 + wmu * 32 * MB + i * 32 + 8 * (r / 4) + (r % 4));
                const float v0 = __fmul_rn(acc[i][0][r], e[0]), v1 = __fmul_rn(acc[i][1][r], e[1]);
                if constexpr (EP == SEPAL_HIP_SWIGLU && YT == kYPairs) {
                    store_h<YT>(p.y, row + 4 * (lane / 32), p.ld_y, n0 / 2 + 64 * ibu + 32 * hhu + lane % 32, swiglu_fast(v0, v1));
                } else if constexpr (EP == SEPAL_HIP_SWIGLU) {
                    char* const rp = yb + (row * p.ld_y + n0 / 2 + 64 * ibu + 32 * hhu) * ES;
                    store_out<YT>(rp + voff, 0, swiglu_fast(v0, v1));
                } else {
                    char* const rp0 = yb + (row * p.ld_y + n0 + 32 * (4 * ibu + hhu)) * ES;
                    char* const rp1 = yb + (row * p.ld_y + n0 + 32 * (4 * ibu + 2 + hhu)) * ES;
                    put_plain<EP, YT>(rp0 + voff, 0, v0);
                    put_plain<EP, YT>(rp1 + voff, 0, v1);
                }
            }
        }
        if constexpr (OVERLAP) wait_vmcnt<0>();
        return;
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + wm * 32 * MB + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
            if (row >= p.t) continue;
            const float v0 = __fmul_rn(acc[i][0][r], e[0]), v1 = __fmul_rn(acc[i][1][r], e[1]);
            if constexpr (EP == SEPAL_HIP_SWIGLU) {
                const int f = n0 / 2 + 64 * ib + 32 * hh + lane % 32;
                if (2 * f < p.n) store_h<YT>(p.y, static_cast<std::size_t>(row), p.ld_y, f, swiglu_fast(v0, v1));
            } else {
                if (col[0] < p.n) put_plain<EP, YT>(p.y, static_cast<std::size_t>(row) * p.ld_y + col[0], v0);
                if (col[1] < p.n) put_plain<EP, YT>(p.y, static_cast<std::size_t>(row) * p.ld_y + col[1], v1);
            }
        }
    }
    if constexpr (OVERLAP) wait_vmcnt<0>();
}

template <int XT, int EP, int YT, int MB, int SPLIT, bool SK>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) gemm_big3(const BigParams p) {
    // MB m-blocks of 32 rows per wave: tiles of BM3 = 64 MB rows (256, or 128 for the tail rows of a launch).
    // SK: the dense order (only block tiles with rows to do), the K range split over BigParams::splits blocks (1: the
    // whole K, no hand-off).
    // SPLIT 2: X is a float32 operand as a bf16 hi + lo pair, stored as one bf16 row of 2K values (64-value chunk j of
    // k is chunk 2j (hi) and 2j + 1 (lo)); steps 2j and 2j + 1 multiply the same weights, so p.k counts the 2K values
    // and the weight offset of step kt is kt / 2 chunks.
    static_assert(SPLIT == 1 || (SPLIT == 2 && XT == SEPAL_HIP_BF16), "the hi + lo form is bf16");
    constexpr int NW = 8, BN = 256, K3 = 64, SUB = K3 / 16, SPG = SPLIT * 128 / K3, BM3 = 64 * MB;
    constexpr int XSTAGE = BM3 * K3 * 2, WSTAGE = (BN / 32) * SUB * 1024;
    constexpr int XLD = XSTAGE / 16 / (64 * NW);       // X direct loads per thread per step (4)
    constexpr int WLD = BN * K3 / 16 / (64 * NW);      // W 16-byte chunks per thread per step (2)
    __shared__ __align__(1024) unsigned char xs0[XSTAGE], xs1[XSTAGE], xs2[XSTAGE], ws0[WSTAGE], ws1[WSTAGE];
    const auto xstage = [&](auto it) -> lds_byte* {
        constexpr int i = decltype(it)::value;
        if constexpr (i == 0) return (lds_byte*)xs0;
        else if constexpr (i == 1) return (lds_byte*)xs1;
        else return (lds_byte*)xs2;
    };
    const auto wstage = [&](auto it) -> lds_byte* {
        if constexpr (decltype(it)::value == 0) return (lds_byte*)ws0;
        else return (lds_byte*)ws1;
    };

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int wm = wave % 2, wn = wave / 2;
    // The dense order (SK): logical id -> block tile sub0 + id / S (sub-rows fastest, so consecutive ids share
    // the weight tile) and split id mod S; the splits of one block tile take consecutive logical ids, which stay on
    // one XCD (shared L2). Otherwise MB 4: one logical 256 x 256 tile per block; MB 2 or 1: block b is part b / count
    // (BM3 rows) of tile id0 + b % count; a part wholly past T has nothing to do.
    int tm, tn, m0;
    int sub = 0, split = 0;
    if constexpr (SK) {
        const int logical = xcd_id(blockIdx.x, static_cast<int>(gridDim.x));
        sub = logical / p.splits;
        split = logical % p.splits;
        const int sg = p.sub0 + sub;
        m0 = (sg % p.sub_m) * BM3;
        tn = sg / p.sub_m;
    } else if constexpr (MB == 4) {
        tile_from_id(p.id0 + xcd_id(blockIdx.x, p.count), p.tiles_m, p.tiles_n, tm, tn);
        m0 = tm * 256;
    } else {
        const int b = blockIdx.x;
        tile_from_id(p.id0 + b % p.count, p.tiles_m, p.tiles_n, tm, tn);
        m0 = tm * 256 + (b / p.count) * BM3;
        if (m0 >= p.t) return;
    }
    const int n0 = tn * BN;
    // this block's whole groups [g0, g1) of the k range, as steps [kbase, kbase + KT)
    const int all_groups = p.k / K3 / SPG;
    const int nsplit = SK ? p.splits : 1;
    const int g0 = split * all_groups / nsplit, g1 = (split + 1) * all_groups / nsplit;
    const int kbase = g0 * SPG;
    const int KT = (g1 - g0) * SPG;

    // Loads go through buffer descriptors: 32-bit lane offsets, the step and the instruction in the scalar offset, and
    // rows past T or N read as zero (past num_records); the launcher checks that every offset fits.
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned short*>(p.x), 0, static_cast<int>(p.x_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<signed char*>(p.w), 0, static_cast<int>(p.w_bytes), 0x00020000);
    // X: direct load i of wave w fills LDS kilobyte w + 8 i = rows 8 w + 64 i + {0..7}; lane l writes slot l % 8 of row
    // 8 w + 64 i + l / 8, which holds chunk (l % 8) ^ ((row / 2) & 7) = (l % 8) ^ ((4 w + l / 16) & 7)
    int xoff;
    {
        const int r = 8 * wave + lane / 8, c = (lane % 8) ^ ((4 * wave + lane / 16) & 7);
        xoff = (m0 + r) * static_cast<int>(p.ld_x) * 2 + 16 * c;
    }
    // X fragment reads: lane l of m-block mb, substep st reads row 32 mb + l % 32, chunk 2 st + l / 32
    int rx[SUB];
#pragma unroll
    for (int st = 0; st < SUB; ++st) rx[st] = (lane % 32) * 128 + 16 * ((2 * st + lane / 32) ^ ((lane / 2) & 7));
    // W: instruction i of wave w covers rows 32 w + 16 i + {0, 1, 8, 9} + 2 (lane / 16) (n-block w); a lane loads one
    // substep's 16 bytes and writes them widened as the fragment's two halves (slots L and L + 32)
    int woff, wdst0, wdst1;
    {
        const int q = lane % 4, u = (lane / 4) % 4;
        const int L = (u & 1) + 8 * (u >> 1) + 2 * (lane / 16);  // row within the n-block for i = 0 (+16 i)
        woff = (n0 + 32 * wave + L) * static_cast<int>(p.ld_w) + 16 * q;
        const int frag = (wave * SUB + q) * 1024;
        wdst0 = frag + 16 * (L ^ (2 * q));             // + 256 i
        wdst1 = frag + 16 * ((L + 32) ^ (2 * q + 1));  // + 256 i
    }
    int rd[SUB];  // this lane's slot in a W fragment of substep st
#pragma unroll
    for (int st = 0; st < SUB; ++st) rd[st] = 16 * (lane ^ ((2 * st + lane / 32) & 7));

    const int ib = wn / 2, hh = wn % 2;
    const int nbj[2] = {4 * ib + hh, 4 * ib + 2 + hh};
    int col[2];
    const float* ssrc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        col[j] = n0 + 32 * nbj[j] + lane % 32;
        ssrc[j] = p.s + static_cast<std::size_t>(min(col[j], p.n - 1)) * p.ld_s;
    }

    struct Regs {
        u32x4 w[WLD];
    };
    float snext[2];
    const int xstride = 64 * static_cast<int>(p.ld_x) * 2, wstride = 16 * static_cast<int>(p.ld_w);
    const auto issue_x = [&](int kt, lds_byte* xd) {
#pragma unroll
        for (int i = 0; i < XLD; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (__attribute__((address_space(3))) void*)(xd + (wave + 8 * i) * 1024), 16,
                                                     xoff, (kbase + kt) * K3 * 2 + i * xstride, 0, 0);
    };
    const auto issue_w = [&](int kt, Regs& r) {
#pragma unroll
        for (int i = 0; i < WLD; ++i)
            r.w[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wres, woff, ((kbase + kt) / SPLIT) * K3 + i * wstride, 0));
    };
    const auto issue_scales = [&](int g) {
        snext[0] = ssrc[0][g0 + g];
        snext[1] = ssrc[1][g0 + g];
    };
    const auto stage_w = [&](lds_byte* wd, const Regs& r) {
#pragma unroll
        for (int i = 0; i < WLD; ++i) {
            unsigned o[8];
            widen16<XT>(r.w[i], o);
            *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(wd + wdst0 + 256 * i) = u32x4{o[0], o[1], o[2], o[3]};
            *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(wd + wdst1 + 256 * i) = u32x4{o[4], o[5], o[6], o[7]};
        }
    };
    // the wait leaves the loads issued by the current step in flight (at most 2 scales, XLD X, WLD W) and covers every
    // earlier one, among them the next step's X
    const auto barrier = [&]() {
        asm volatile("" ::: "memory");
        wait_vm_lgkm0<2 + XLD + WLD>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    f32x16 acc[MB][2];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int groups = KT / SPG;
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    Regs r0, r1;
    issue_scales(0);
    issue_x(0, xstage(I0{}));
    issue_x(min(1, KT - 1), xstage(I1{}));
    __builtin_amdgcn_sched_barrier(0);
    issue_w(0, r0);
    issue_w(min(1, KT - 1), r1);
    __builtin_amdgcn_sched_barrier(0);
    stage_w(wstage(I0{}), r0);
    asm volatile("" ::: "memory");
    wait_vm_lgkm0<WLD>();  // everything but step 1's W (X of steps 0 and 1 included)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // the Horner state (the first step's factor multiplies zero accumulators)
    float e[2] = {1.0f, 1.0f}, emax[2] = {0.0f, 0.0f};

    // Step kt (j = kt mod 6): at a group's first step the Horner rescale with the group's scales (loaded one group
    // ahead), then the next group's scales are issued; the direct X loads of step kt + 2 into X stage (j + 2) mod 3 (last
    // read by step kt - 1); step kt + 2's W into the registers freed by step kt; the multiply of step kt from X stage
    // j mod 3 and W stage j mod 2; step kt + 1's W into its stage; one barrier. Loads past the end repeat the last step
    // (clamped) and land in stages nothing reads again.
    const auto step = [&](int kt, auto jt) {
        constexpr int j = decltype(jt)::value;
        constexpr bool first = j % SPG == 0;
        Regs& r_next = j % 2 == 0 ? r1 : r0;
        Regs& r_free = j % 2 == 0 ? r0 : r1;
        const lds_byte* xs = xstage(std::integral_constant<int, j % 3>{});
        const lds_byte* ws = wstage(std::integral_constant<int, j % 2>{});
        float ratio[2] = {1.0f, 1.0f};
        if constexpr (first) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                ratio[q] = horner_step(snext[q], e[q], emax[q]);
            }
            issue_scales(min(kt / SPG + 1, groups - 1));
        }
        issue_x(min(kt + 2, KT - 1), xstage(std::integral_constant<int, (j + 2) % 3>{}));
        __builtin_amdgcn_sched_barrier(0);
        issue_w(min(kt + 2, KT - 1), r_free);
        // keep the loads at the top of the step, in this order: the wait for a step's operands then leaves the later
        // steps' loads in flight
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int st = 0; st < SUB; ++st) {
            u32x4 a[MB], b[2];
#pragma unroll
            for (int i = 0; i < MB; ++i)
                a[i] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(xs + (wm * MB + i) * 4096 + rx[st]);
#pragma unroll
            for (int q = 0; q < 2; ++q)
                b[q] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(ws + (nbj[q] * SUB + st) * 1024 + rd[st]);
#pragma unroll
            for (int i = 0; i < MB; ++i)
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    // a group's Horner rescale of each accumulator block right before its first MFMA of the group:
                    // the multiplies of one block overlap the MFMA of the previous one
                    if constexpr (first)
                        if (st == 0) acc[i][q] = acc[i][q] * ratio[q];
                    acc[i][q] = mfma32<XT>(a[i], b[q], acc[i][q]);
                }
        }
        if constexpr (first) {
            // the first substep's fragment reads, then each block's 16 rescale multiplies and its MFMA, in turn
            __builtin_amdgcn_sched_group_barrier(0x100, MB + 2, 0);
#pragma unroll
            for (int q = 0; q < 2 * MB; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
        }
        stage_w(wstage(std::integral_constant<int, (j + 1) % 2>{}), r_next);
        barrier();
    };
    // the loop body is three groups (6 SPLIT steps: a multiple of the 3 X stages and 2 W stages), then at most two
    // whole groups remain
    constexpr int U = 3 * SPG;
    const auto steps = [&]<int... J>(int k0, std::integer_sequence<int, J...>) {
        (step(k0 + J, std::integral_constant<int, J>{}), ...);
    };
    int kt = 0;
    for (; kt + U <= KT; kt += U) steps(kt, std::make_integer_sequence<int, U>{});
    if (kt + SPG <= KT) {
        steps(kt, std::make_integer_sequence<int, SPG>{});
        if (kt + 2 * SPG <= KT) {
            [&]<int... J>(std::integer_sequence<int, J...>) {
                (step(kt + SPG + J, std::integral_constant<int, SPG + J>{}), ...);
            }(std::make_integer_sequence<int, SPG>{});
        }
    }
    // no direct load may still be writing LDS when the block ends
    wait_vmcnt<0>();

    if constexpr (SK) if (p.splits > 1) {
        // This split's sums s_g P_g over its groups, value v of thread tid at part[((sub S + split) 32 MB + v) 512 + tid].
        // The hand-off between the splits of a block tile uses no device-wide fence (on gfx950 one writes back and
        // invalidates the L2 of the XCD): the partials are written and read with device-scope relaxed atomics, which go
        // to the device coherence point; each thread waits for its stores to complete before the barrier, and only
        // then does one thread count the block in. The last block to arrive adds the S partials in split order (its
        // own read back like the others), so the result does not depend on the arrival order.
        if (p.planes) {
            BigParams q = p;
            q.y = p.part + static_cast<std::size_t>(split) * p.t * p.n;
            q.ld_y = static_cast<std::size_t>(p.n);
            tile_epilogue<SEPAL_HIP_STORE, SEPAL_HIP_F32, MB>(q, acc, e, m0, n0, wave, lane);
            return;
        }
        constexpr int NV = MB * 32;
        float* mine = p.part + (static_cast<std::size_t>(sub) * p.splits + split) * NV * 512 + tid;
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    __hip_atomic_store(mine + ((i * 2 + q) * 16 + r) * 512, __fmul_rn(acc[i][q][r], e[q]), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);  // also every direct load of this wave: after the barrier no load writes LDS
        __syncthreads();
        unsigned* last = reinterpret_cast<unsigned*>(xs0);  // the stages are free now (the LDS is full)
        if (tid == 0)
            *last = __hip_atomic_fetch_add(&p.counters[sub], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                            static_cast<unsigned>(p.splits - 1) ? 1u : 0u;
        __syncthreads();
        if (*last == 0u) return;
        // C partials' loads in flight at a time (128 values per thread), then added in split order
        constexpr int C = 4 / MB;
        const float* base = p.part + static_cast<std::size_t>(sub) * p.splits * NV * 512 + tid;
        for (int sp0 = 0; sp0 < p.splits; sp0 += C) {
            float v[C][NV];
#pragma unroll
            for (int c = 0; c < C; ++c) {
                const float* src = base + static_cast<std::size_t>(min(sp0 + c, p.splits - 1)) * NV * 512;
#pragma unroll
                for (int u = 0; u < NV; ++u) v[c][u] = __hip_atomic_load(src + u * 512, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int c = 0; c < C; ++c)
                if (sp0 + c < p.splits) {
#pragma unroll
                    for (int i = 0; i < MB; ++i)
#pragma unroll
                        for (int q = 0; q < 2; ++q)
#pragma unroll
                            for (int r = 0; r < 16; ++r) {
                                const float x = v[c][(i * 2 + q) * 16 + r];
                                acc[i][q][r] = sp0 + c == 0 ? x : __fadd_rn(acc[i][q][r], x);
                            }
                }
        }
        if (tid == 0) __hip_atomic_store(&p.counters[sub], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        e[0] = e[1] = 1.0f;  // the sums are final values (x 1 is exact)
    }

    tile_epilogue<EP, YT, MB>(p, acc, e, m0, n0, wave, lane);
}

// ---- large-M kernel, two wave groups in alternation (gemm_pp) --------------------------------------------------------
//
// The tile, waves, outputs, k order and Horner chain of gemm_big3<MB> (so the same bits), scheduled so that the
// MFMA units, the LDS and the VALU work at the same time instead of in turn. Waves 0-3 (group A, one per SIMD) and
// 4-7 (group B) each alternate two slots per 64-wide step, separated by block barriers: L(k) issues the stage loads
// of a later step and reads 20 of step k's 24 operand fragments (every W fragment, X of substeps 0 to 2); M(k) issues
// the step's 32 MFMAs (at a group's first step each block's Horner rescale right before its first MFMA) and reads X of
// substep 3 behind the MFMAs of the earlier substeps (all 24 fragments at once would not fit the registers).
// Group B runs one slot behind group A (one extra barrier at its start, one at A's end), so in every slot one wave of
// each SIMD multiplies while the other mostly reads. Slot 2k: A L(k), B M(k - 1); slot 2k + 1: A M(k), B L(k). An X
// stage is read until the end of group B's M(k), slot 2k + 2, and reloaded from slot 2k + 3.
// The full-tile launch is persistent (one block per CU over its XCD's tiles; the next tile's first loads are issued
// before the current tile's epilogue). Stages: X of step k in X stage k mod 3, W of step k in W stage k mod 2 (from
// the weight image). Group A issues all
// W loads (step k + 1 at the start of L(k), due by the barrier that ends slot 2k + 1), group B all X loads (step k + 2
// at the start of its L(k), slot 2k + 1, due by the barrier that ends slot 2k + 3). A stage is reloaded only after
// the barrier that follows both groups' reads of it, and every L slot waits for its reads before its barrier.
template <int XT, int EP, int YT, int MB, int SPLIT>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) gemm_pp(const BigParams p) {
    // MB m-blocks of 32 rows per wave: tiles of BM3 = 64 MB rows (256, or 128 for the last round of a launch)
    static_assert(SPLIT == 1 || (SPLIT == 2 && XT == SEPAL_HIP_BF16), "the hi + lo form is bf16");
    static_assert(MB == 4 || MB == 2, "256- or 128-row tiles");
    constexpr int BN = 256, K3 = 64, SUB = K3 / 16, SPG = SPLIT * 128 / K3, BM3 = 64 * MB;
    constexpr int XSTAGE = BM3 * K3 * 2, WSTAGE = (BN / 32) * SUB * 1024;
    constexpr int LDGX = XSTAGE / 1024 / 4, LDGW = WSTAGE / 1024 / 4;  // direct loads per wave of B (X) / A (W) per step
    __shared__ __align__(1024) unsigned char xs0[XSTAGE], xs1[XSTAGE], xs2[XSTAGE], ws0[WSTAGE], ws1[WSTAGE];
    const auto xstage = [&](auto it) -> lds_byte* {
        constexpr int i = decltype(it)::value;
        if constexpr (i == 0) return (lds_byte*)xs0;
        else if constexpr (i == 1) return (lds_byte*)xs1;
        else return (lds_byte*)xs2;
    };
    const auto wstage = [&](auto it) -> lds_byte* {
        if constexpr (decltype(it)::value == 0) return (lds_byte*)ws0;
        else return (lds_byte*)ws1;
    };

    const int tid = threadIdx.x, lane = tid % 64;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int wg = wave % 4;            // the wave's index in its group
    const bool group_b = wave >= 4;
    const int wm = wave % 2, wn = wave / 2;
    // MB 4 (persistent): one block per CU; block b works through the contiguous range [lo, hi) of logical tiles of its
    // XCD (b mod 8), every (gridDim.x / 8)-th from lo + b / 8, so the XCD's blocks run consecutive tiles at a time
    // (they share its L2). MB 2: block b is half b / count of tile id0 + b % count (a half wholly past T has nothing to
    // do, and leaves before any barrier).
    int tm, tn, m0, n0, cur = 0, stride = 1, hi = 1;
    if constexpr (MB == 2) {
        // the blocks past the halves widen the stack's next weight image (they share no barrier with the others)
        const int halves = 2 * p.count;
        if (static_cast<int>(blockIdx.x) >= halves) {
            widen_range(p.jw, p.j_ld, p.j_n, p.j_wsteps, p.j_tiles_n, p.j_img, p.j_f16 != 0,
                        (blockIdx.x - halves) * 512ull + threadIdx.x, static_cast<std::size_t>(p.j_blocks) * 512);
            return;
        }
    }
    if constexpr (MB == 4) {
        const int nx = static_cast<int>(gridDim.x) / 8, xcd = blockIdx.x % 8;
        const int q = p.count / 8, r = p.count % 8;
        const int lo = xcd * q + min(xcd, r);
        hi = lo + q + (xcd < r ? 1 : 0);
        cur = lo + static_cast<int>(blockIdx.x) / 8;
        stride = nx;
        if (cur >= hi) return;
    }
    const auto tile_at = [&](int id) __attribute__((always_inline)) {
        if constexpr (MB == 4) {
            tile_from_id(p.id0 + id, p.tiles_m, p.tiles_n, tm, tn);
            m0 = tm * 256;
        } else {
            const int bb = blockIdx.x;
            tile_from_id(p.id0 + bb % p.count, p.tiles_m, p.tiles_n, tm, tn);
            m0 = tm * 256 + (bb / p.count) * BM3;
        }
        n0 = tn * BN;
    };
    tile_at(cur);
    if (m0 >= p.t) return;
    const int KT = p.k / K3, groups = KT / SPG;

    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned short*>(p.x), 0, static_cast<int>(p.x_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t wires = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(p.wimg), 0, static_cast<int>(p.wimg_bytes), 0x00020000);
    // X (group B): direct load i of group wave g fills LDS kilobyte g + 4 i = rows 8 g + 32 i + {0..7}; lane l writes
    // slot l % 8 of row 8 g + 32 i + l / 8, which holds chunk (l % 8) ^ ((row / 2) & 7) = (l % 8) ^ ((4 g + l / 16) & 7)
    const int xrow = 8 * wg + lane / 8, xchunk = (lane % 8) ^ ((4 * wg + lane / 16) & 7);
    const int xstride = 32 * static_cast<int>(p.ld_x) * 2;
    int rx[SUB];
#pragma unroll
    for (int st = 0; st < SUB; ++st) rx[st] = (lane % 32) * 128 + 16 * ((2 * st + lane / 32) ^ ((lane / 2) & 7));
    const int ib = wn / 2, hh = wn % 2;
    const int nbj[2] = {4 * ib + hh, 4 * ib + 2 + hh};
    // the scales through a buffer descriptor: a 32-bit byte offset per lane and column, the group in the scalar offset
    const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.s), 0, static_cast<int>(static_cast<std::size_t>(p.n) * p.ld_s * 4), 0x00020000);
    // (columns past N read as 0: a zero scale keeps the Horner state; the second column is 64 columns on)
    const int soff1 = 64 * static_cast<int>(p.ld_s) * 4;

    // The wave's load role, chosen once (no branch in the loop): group B loads X, group A the weight image. Load i of
    // group wave g fills LDS kilobyte g + 4 i of the stage.
    // the tile's offsets (set_tile)
    int wimg_tile, lvoff, soff;
    const auto set_tile = [&]() __attribute__((always_inline)) {
        wimg_tile = tn * p.wsteps;
        lvoff = group_b ? (m0 + xrow) * static_cast<int>(p.ld_x) * 2 + 16 * xchunk : wg * 1024 + lane * 16;
        soff = (n0 + 32 * nbj[0] + lane % 32) * static_cast<int>(p.ld_s) * 4;
    };
    set_tile();
    const __amdgpu_buffer_rsrc_t lres = group_b ? xres : wires;
    const int lstride = group_b ? xstride : 4096;
    const int nld = group_b ? LDGX : LDGW;
    const auto issue = [&](int soff, lds_byte* dst) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < LDGW; ++i)
            if (LDGX == LDGW || i < nld)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(lres, (__attribute__((address_space(3))) void*)(dst + (wg + 4 * i) * 1024), 16,
                                                         lvoff, soff + i * lstride, 0, 0);
    };
    const auto x_soff = [&](int kt) __attribute__((always_inline)) { return kt * K3 * 2; };
    const auto w_soff = [&](int kt) __attribute__((always_inline)) { return (wimg_tile + kt / SPLIT) * WSTAGE; };
    float snext[2];
    const auto issue_scales = [&](int g) __attribute__((always_inline)) {
        snext[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sres, soff, 4 * g, 0));
        snext[1] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sres, soff, 4 * g + soff1, 0));
    };
    const auto barrier = [&]() __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };

    f32x16 acc[MB][2];
    float e[2], emax[2];
    u32x4 a[3][MB], b[SUB][2];  // X fragments of substeps 0, 1, 2 (then 3 in the first), W of every substep

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // a tile's first loads: the first group's scales, X of steps 0 and 1 (group B), W of step 0 (group A)
    const auto first_loads = [&]() __attribute__((always_inline)) {
        issue_scales(0);
        if (group_b) {
            issue(x_soff(0), xstage(I0{}));
            issue(x_soff(min(1, KT - 1)), xstage(I1{}));
        } else {
            issue(w_soff(0), wstage(I0{}));
        }
    };
    first_loads();
    wait_vm_lgkm0<0>();

    // Step kt (j = kt mod 6): slot L then slot M, each ended by a barrier.
    const auto step = [&](int kt, auto jt) __attribute__((always_inline)) {
        constexpr int j = decltype(jt)::value;
        constexpr bool first = j % SPG == 0;
        const lds_byte* xs = xstage(std::integral_constant<int, j % 3>{});
        const lds_byte* ws = wstage(std::integral_constant<int, j % 2>{});
        // ---- L(kt): loads of later steps, this step's fragments (the Horner factors at a group's first step)
        float ratio[2] = {1.0f, 1.0f};
        if constexpr (first) {
#pragma unroll
            for (int q = 0; q < 2; ++q) ratio[q] = horner_step(snext[q], e[q], emax[q]);
        }
        issue(group_b ? x_soff(min(kt + 2, KT - 1)) : w_soff(min(kt + 1, KT - 1)),
              group_b ? xstage(std::integral_constant<int, (j + 2) % 3>{}) : wstage(std::integral_constant<int, (j + 1) % 2>{}));
        // the next group's scales after the stage loads (needed two steps later)
        if constexpr (first) issue_scales(min(kt / SPG + 1, groups - 1));
        __builtin_amdgcn_sched_barrier(0);
        const auto read_x = [&](int st, int sl) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < MB; ++i)
                a[sl][i] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(xs + (wm * MB + i) * 4096 + rx[st]);
        };
        // every W fragment of the step and the X fragments of substeps 0, 1 and 2 (those of substep 3 are read in the
        // M slot, into the registers substep 0 frees: the X stage is reloaded only two slots after the M slot)
#pragma unroll
        for (int st = 0; st < SUB; ++st)
#pragma unroll
            for (int q = 0; q < 2; ++q)
                b[st][q] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(ws + (nbj[q] * SUB + st) * 1024 + 16 * lane);
        read_x(0, 0);
        read_x(1, 1);
        read_x(2, 2);
        // the reads are complete before the barrier (a stage is reloaded right after the barrier that follows them);
        // this slot's stage loads and scales stay in flight (every older load completed at the end of the wave's
        // previous M slot)
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        wait_vm_lgkm0<63>();
        barrier();
        // ---- M(kt): the step's MFMAs; block bl = (i, q) = (bl / 2, bl % 2)
        const auto mma = [&](int bl, int st, int sl) __attribute__((always_inline)) {
            acc[bl / 2][bl % 2] = mfma32<XT>(a[sl][bl / 2], b[st][bl % 2], acc[bl / 2][bl % 2]);
        };
        if constexpr (first) {
            // each block's Horner rescale, then its substep 0 MFMA and the previous block's substep 1 MFMA: the two
            // MFMAs cover the next block's 16 multiplies
#pragma unroll
            for (int bl = 0; bl < 2 * MB; ++bl) {
                acc[bl / 2][bl % 2] = acc[bl / 2][bl % 2] * ratio[bl % 2];
                mma(bl, 0, 0);
                if (bl > 0) mma(bl - 1, 1, 1);
            }
            mma(2 * MB - 1, 1, 1);
            read_x(3, 0);
#pragma unroll
            for (int bl = 0; bl < 2 * MB; ++bl) mma(bl, 2, 2);
#pragma unroll
            for (int bl = 0; bl < 2 * MB; ++bl) mma(bl, 3, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
            for (int bl = 1; bl < 2 * MB; ++bl) {
                __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, MB, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4 * MB, 0);
        } else {
            // substep 0, then substep 3's X reads behind substeps 1 and 2
#pragma unroll
            for (int bl = 0; bl < 2 * MB; ++bl) mma(bl, 0, 0);
            read_x(3, 0);
#pragma unroll
            for (int st = 1; st < SUB; ++st)
#pragma unroll
                for (int bl = 0; bl < 2 * MB; ++bl) mma(bl, st, st % 3);
            __builtin_amdgcn_sched_group_barrier(0x008, 2 * MB, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, MB, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 6 * MB, 0);
        }
        // group A's W loads of step kt + 1 are due (group A reads that stage in the next slot); group B's X loads of
        // step kt + 2 complete here too, a slot before they are due
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        wait_vm_lgkm0<0>();
        barrier();
    };
    constexpr int U = 3 * SPG;
    const auto steps = [&]<int... J>(int k0, std::integer_sequence<int, J...>) __attribute__((always_inline)) {
        (step(k0 + J, std::integral_constant<int, J>{}), ...);
    };
    // Tile loop. Per tile the barriers balance: group A 1 + 2 KT + 1, group B 1 + 1 + 2 KT. After the last one every
    // wave has read the tile's stages for the last time and waited for every load it issued, so the next tile's first
    // loads go out before this tile's epilogue, whose values are computed while they fly (MB 4).
    for (;;) {
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        e[0] = e[1] = 1.0f;
        emax[0] = emax[1] = 0.0f;
        barrier();
        if (group_b) barrier();  // B runs one slot behind A
        int kt = 0;
        for (; kt + U <= KT; kt += U) steps(kt, std::make_integer_sequence<int, U>{});
        if (kt + SPG <= KT) {
            steps(kt, std::make_integer_sequence<int, SPG>{});
            if (kt + 2 * SPG <= KT) {
                [&]<int... J>(std::integer_sequence<int, J...>) __attribute__((always_inline)) {
                    (step(kt + SPG + J, std::integral_constant<int, SPG + J>{}), ...);
                }(std::make_integer_sequence<int, SPG>{});
            }
        }
        if (!group_b) barrier();  // matches group B's extra barrier
        const int mc = m0, nc = n0;
        cur += stride;
        const bool more = MB == 4 && cur < hi;
        if (more) {
            tile_at(cur);
            set_tile();
            first_loads();
        }
        if constexpr (MB == 4) tile_epilogue<EP, YT, MB, true>(p, acc, e, mc, nc, wave, lane);
        else tile_epilogue<EP, YT, MB>(p, acc, e, mc, nc, wave, lane);
        if (!more) break;
    }
}

template <int WN>
constexpr std::size_t lds_bytes() {
    return static_cast<std::size_t>(STAGES) * ((BM / 32) * (BK / 16) + (64 * WN / 32) * (BK / 16)) * 1024;
}

} // namespace v2

// ---- launch ----------------------------------------------------------------------------------------------------------

template <int XT, int EP, int YT, int WN>
void launch_big2(const BigParams& p, hipStream_t stream) {
    const auto kernel = v2::gemm_big2<XT, EP, YT, WN>;
    const std::size_t lds = v2::lds_bytes<WN>();
    static_assert(v2::lds_bytes<WN>() <= (160u << 10), "LDS of one CU");
    raise_dynamic_lds(reinterpret_cast<const void*>(kernel), lds, "gemm_w8g large-M");
    kernel<<<dim3(p.tiles_m * p.tiles_n), dim3(128 * WN), lds, stream>>>(p);
}

// Compute units of the current device (cached per device).
inline int device_cus() {
    static std::atomic<int> cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) throw LaunchError("gemm_w8g: hipGetDevice failed");
    if (dev < 64) {
        const int known = cached[dev].load(std::memory_order_relaxed);
        if (known > 0) return known;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        throw LaunchError("gemm_w8g: device query failed");
    if (dev < 64) cached[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

// The planes of a split-K launch added in split order, then the epilogue: the additions and epilogue operations of
// the hand-off (sum = plane 0, then sum + plane s; x 1; the tile epilogue's conversion), so the same bits. A thread
// takes 4 consecutive outputs of one row: Store / Add columns c..c+3, or SwiGLU features f..f+3, whose gate and up
// columns are 128 (f / 64) + f % 64 and 64 past it (the gate/up interleave of a 256-column tile). VEC: n % 4 == 0
// (16-byte plane reads).
template <int EP, int YT, bool VEC>
__global__ void __launch_bounds__(256) planes_sum_kernel(const float* __restrict__ part, int splits, int t, int n, void* y,
                                                         std::size_t ld_y) {
    const int outs = EP == SEPAL_HIP_SWIGLU ? n / 2 : n;
    const int per_row = (outs + 3) / 4;
    const long id = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= static_cast<long>(t) * per_row) return;
    const int row = static_cast<int>(id / per_row), c0 = static_cast<int>(id % per_row) * 4;
    const std::size_t plane = static_cast<std::size_t>(t) * n;
    const auto sum4 = [&](int col, float (&s)[4]) {
        const float* src = part + static_cast<std::size_t>(row) * n + col;
        for (int sp = 0; sp < splits; ++sp, src += plane) {
            float v[4];
            if constexpr (VEC) {
                const float4 f = *reinterpret_cast<const float4*>(src);
                v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = col + j < n ? src[j] : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) s[j] = sp == 0 ? v[j] : __fadd_rn(s[j], v[j]);
        }
    };
    if constexpr (EP == SEPAL_HIP_SWIGLU) {
        float g[4], u[4];
        const int gc = 128 * (c0 / 64) + c0 % 64;
        sum4(gc, g);
        sum4(gc + 64, u);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (c0 + j < outs) store_h<YT>(y, static_cast<std::size_t>(row), ld_y, c0 + j, swiglu_fast(__fmul_rn(g[j], 1.0f), __fmul_rn(u[j], 1.0f)));
    } else {
        float s[4];
        sum4(c0, s);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (c0 + j < outs) put_plain<EP, YT>(y, static_cast<std::size_t>(row) * ld_y + c0 + j, __fmul_rn(s[j], 1.0f));
    }
}

template <int EP, int YT>
void launch_planes_sum(const float* part, int splits, int t, int n, void* y, std::size_t ld_y, hipStream_t stream) {
    const int outs = EP == SEPAL_HIP_SWIGLU ? n / 2 : n;
    const long threads = static_cast<long>(t) * ((outs + 3) / 4);
    const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
    if (n % 4 == 0) planes_sum_kernel<EP, YT, true><<<grid, dim3(256), 0, stream>>>(part, splits, t, n, y, ld_y);
    else planes_sum_kernel<EP, YT, false><<<grid, dim3(256), 0, stream>>>(part, splits, t, n, y, ld_y);
}

template <int XT, int EP, int YT, int MB, int SPLIT>
void launch_big3(const BigParams& p, hipStream_t stream) {
    const int blocks = p.dense ? p.nsub * p.splits : p.count * (256 / (64 * MB));
    if (p.dense) v2::gemm_big3<XT, EP, YT, MB, SPLIT, true><<<dim3(blocks), dim3(512), 0, stream>>>(p);
    else v2::gemm_big3<XT, EP, YT, MB, SPLIT, false><<<dim3(blocks), dim3(512), 0, stream>>>(p);
}

// The weight image of gemm_pp: for every 256-column tile tn and weight step ks (64 values of k), the 32 KB
// W stage in the order the fragment reads use it. Kilobyte 4 nb + st holds n-block nb (32 columns) at substep st (16
// values of k); in it, lane l's 16 bytes are column 32 nb + l % 32 at k 16 st + 8 (l / 32) .. + 7, widened exactly to
// the MFMA type (the same values the waves would widen into the stage). Columns past N are zero. One thread widens one
// 16-byte chunk of one weight row (widen_range).
__global__ void __launch_bounds__(256) widen_image_kernel(const signed char* __restrict__ w, std::size_t ld_w, int n,
                                                          int wsteps, int tiles_n, unsigned char* __restrict__ img, int f16) {
    widen_range(w, ld_w, n, wsteps, tiles_n, img, f16 != 0, blockIdx.x * 256ull + threadIdx.x, static_cast<std::size_t>(gridDim.x) * 256);
}

// Bytes of the weight image for an N x K multiply (0 when it would not fit 32-bit offsets).
inline std::size_t image_bytes(std::size_t n, std::size_t k) {
    const std::size_t b = (n + 255) / 256 * (k / 64) * 32768;
    return b < (std::size_t{1} << 31) ? b : 0;
}

// One streaming pass that widens an N x K int8 weight matrix into its image (binary16 or bf16).
inline void launch_widen(const std::int8_t* w, std::size_t ld_w, std::size_t n, std::size_t k, bool f16, void* img,
                         hipStream_t stream) {
    const int wsteps = static_cast<int>(k / 64), tiles_n = static_cast<int>((n + 255) / 256);
    const std::size_t items = static_cast<std::size_t>(tiles_n) * (wsteps / 2) * 256 * 8;
    widen_image_kernel<<<static_cast<int>(std::min<std::size_t>((items + 255) / 256, 16384)), 256, 0, stream>>>(
        reinterpret_cast<const signed char*>(w), ld_w, static_cast<int>(n), wsteps, tiles_n, static_cast<unsigned char*>(img),
        f16 ? 1 : 0);
    check_launch("gemm_w8g weight image launch");
}

// Grids of fewer than two rounds of 256 x 256 tiles. The block tile is 64, 128 or 256 rows high (MB 1, 2, 4), and when
// allowed the K range is split over S blocks in whole groups (split-K), by the plan of least modelled time. Every tile
// height runs the same k order and Horner chain per output, so MB does not change a row's bits; a split does (the
// splits' partial sums are added in float32), so callers that need a row's bits independent of the batch keep S = 1
// (config 0).
struct SmallGridPlan {
    int mb = 1, splits = 1;
    bool planes = false;      // split-K through planes and planes_sum_kernel instead of the in-kernel hand-off
    // row split: the floor(T / 256) x 256 leading rows as unsplit 256 x 256 tiles, then the remaining rows as a grid of
    // their own with (mb2, splits2, planes2)
    bool rows = false;
    int mb2 = 1, splits2 = 1;
    bool planes2 = false;
};

// Modelled time (us) of one grid of t rows: fitted to times measured on MI355X (the MLP shapes, M from 65 to 12288,
// every plan): the time per 128-value group of a lone block of 64, 128 or 256 rows (MB 1, 2, 4); the rate at which
// the blocks' operand reads are served; the in-kernel split hand-off, a fixed cost plus the last block's reads of the
// S partials of its tile (one block's coherent reads are slow); or the planes' finisher, a launch plus the S planes
// read and the output written at the rate of a plain streaming kernel. Negative: the plan does not fit the scratch.
inline double grid_cost(long t, int tiles_n, int groups, int mb, int sp, bool planes, int cus) {
    constexpr double us_per_group[5] = {0.0, 1.65, 2.44, 0.0, 4.60};
    constexpr double operand_bytes_per_us = 9.27e6, handoff_us = 5.7, tail_bytes_per_us = 8.8e4;
    constexpr double finish_us = 2.5, stream_bytes_per_us = 3.45e6;
    const int rows = 64 * mb;
    const long subs = (t + rows - 1) / rows * tiles_n;  // block tiles with rows to do
    const double plane = static_cast<double>(t) * tiles_n * 256 * sizeof(float);
    if (sp > 1) {
        if (planes && plane * sp > static_cast<double>(kPartialBytes)) return -1.0;
        if (!planes && (subs * static_cast<long>(sizeof(unsigned)) > static_cast<long>(kCounterBytes) ||
                        static_cast<double>(subs) * sp * rows * 256 * sizeof(float) > static_cast<double>(kPartialBytes)))
            return -1.0;
    }
    const long blocks = subs * sp, rounds = (blocks + cus - 1) / cus;
    const int per_block = (groups + sp - 1) / sp;
    const double compute = static_cast<double>(rounds) * per_block * us_per_group[mb];
    const double operand = static_cast<double>(blocks) * per_block * 128.0 * (2.0 * rows + 256.0) / operand_bytes_per_us;
    double cost = compute > operand ? compute : operand;
    if (sp > 1)
        cost += planes ? finish_us + (sp + 1) * plane / stream_bytes_per_us
                       : handoff_us + static_cast<double>(sp) * rows * 256 * sizeof(float) / tail_bytes_per_us;
    return cost;
}

// The plan of least modelled time: one grid over all rows, or (T above 256 and not a multiple of it) the leading whole
// 256-row tiles unsplit, then the remaining rows as a grid of their own (at M = 896, gate/up 19456 x 2560: 3 x 76
// whole tiles, one round, then 128 rows in 128-row blocks split 3 ways: 107 us against 149-156 us for any one grid;
// the model predicts both within 5%).
inline SmallGridPlan plan_small_grid(const GemmArgs& a, int tiles_n, int groups, bool allow_split) {
    const int cus = device_cus();
    const bool can_split = allow_split && a.scratch != nullptr;
    const auto best_grid = [&](long t, int& mb_out, int& sp_out, bool& pl_out) {
        double best = 1e30;
        for (int mb : {4, 2, 1})
            for (int sp = 1; sp <= 8 && sp <= groups && (sp == 1 || can_split); ++sp)
                for (int pl = 0; pl < (sp > 1 ? 2 : 1); ++pl) {
                    const double c = grid_cost(t, tiles_n, groups, mb, sp, pl != 0, cus);
                    if (c >= 0.0 && c < best) {
                        best = c;
                        mb_out = mb;
                        sp_out = sp;
                        pl_out = pl != 0;
                    }
                }
        return best;
    };
    SmallGridPlan plan;
    const double one = best_grid(static_cast<long>(a.t), plan.mb, plan.splits, plan.planes);
    const long lead = static_cast<long>(a.t) / 256 * 256;
    if (lead > 0 && lead < static_cast<long>(a.t)) {
        constexpr double launch_us = 3.2;
        SmallGridPlan r;
        r.rows = true;
        const double two = grid_cost(lead, tiles_n, groups, 4, 1, false, cus) + launch_us +
                           best_grid(static_cast<long>(a.t) - lead, r.mb2, r.splits2, r.planes2);
        if (two < one) plan = r;
    }
    return plan;
}

// gemm_big3 addresses X and W with 32-bit offsets (rows up to one tile past the end included) and writes SwiGLU outputs
// from whole 256-column tiles. kx: X values per row (K, or 2K for the hi + lo form).
bool big3_takes(const GemmArgs& a, std::size_t kx, std::size_t ld_x) {
    const bool offsets32 = (a.t + 256) * ld_x * 2 < (std::size_t{1} << 31) && (a.n + 256) * a.ld_w < (std::size_t{1} << 31);
    return offsets32 && kx <= ld_x && (a.epilogue != SEPAL_HIP_SWIGLU || a.n % 256 == 0);
}

// Bytes between consecutive rows of Y of type YT (kYPairs: the hi + lo row of 2 ld_y bf16 values).
template <int YT>
constexpr std::size_t y_row_bytes(std::size_t ld_y) {
    return YT == SEPAL_HIP_F32 || YT == kYPairs ? 4 * ld_y : 2 * ld_y;
}

// One gemm_big3 grid over the rows of p (p.tiles_n set): block tiles of 64 mb rows, K split over `splits` blocks
// (through the hand-off, or through planes and planes_sum_kernel).
template <int XT, int EP, int YT, int SPLIT>
void launch_grid(const GemmArgs& a, BigParams p, int mb, int splits, bool planes, hipStream_t stream) {
    p.tiles_m = (p.t + 255) / 256;
    p.id0 = 0;
    p.count = p.tiles_m * p.tiles_n;
    // the dense order (only block tiles with rows to do are launched) for split grids and for blocks below 256 rows
    if (splits > 1 || mb < 4) {
        const int rows = 64 * mb;
        p.dense = 1;
        p.sub_m = (p.t + rows - 1) / rows;
        p.nsub = p.sub_m * p.tiles_n;
        p.splits = splits;
        p.planes = planes ? 1 : 0;
        p.counters = static_cast<unsigned*>(a.scratch);
        p.part = reinterpret_cast<float*>(static_cast<char*>(a.scratch) + kCounterBytes);
    }
    if (mb == 4) launch_big3<XT, EP, YT, 4, SPLIT>(p, stream);
    else if (mb == 2) launch_big3<XT, EP, YT, 2, SPLIT>(p, stream);
    else launch_big3<XT, EP, YT, 1, SPLIT>(p, stream);
    if (splits > 1 && planes) {
        check_launch("gemm_w8g split-K launch");
        launch_planes_sum<EP, YT>(p.part, splits, p.t, p.n, p.y, p.ld_y, stream);
    }
}

template <int XT, int EP, int YT, int SPLIT>
void launch_big(const GemmArgs& a, hipStream_t stream) {
    const std::size_t kx = SPLIT * a.k;  // X values per row
    BigParams p{static_cast<const unsigned short*>(a.x), a.ld_x, reinterpret_cast<const signed char*>(a.w), a.ld_w, a.s, a.ld_s,
                a.y, a.ld_y, static_cast<int>(a.t), static_cast<int>(a.n), static_cast<int>(kx), 0, 0,
                ((a.t - 1) * a.ld_x + kx) * 2, (a.n - 1) * a.ld_w + a.k};
    // 256 x 256 tiles when there are enough of them to fill the chip twice, else 256 x 128
    const int tiles_m = static_cast<int>((a.t + 255) / 256);
    const int tn256 = static_cast<int>((a.n + 255) / 256);
    const bool takes = big3_takes(a, kx, a.ld_x);
    const bool wide = static_cast<long>(tiles_m) * tn256 >= 2 * 256 && (EP != SEPAL_HIP_SWIGLU || a.n % 256 == 0);
    p.tiles_m = tiles_m;
    bool next_done = false;  // the next multiply's image (a stack's) widened by this call's halves launch
    if (wide && takes) {
        // The last, partial round of 256 x 256 tiles is the idle tail of the launch. When it is more than a quarter
        // full and its tiles fit one round as 128 x 256 halves, they go to a second launch of half-height tiles (the
        // logical ids past the full rounds, each as two halves). Both launches run the same k order and Horner chain
        // per output, so a row's bits do not depend on which one computed it.
        const int cus = device_cus();
        const int total = tiles_m * tn256;
        const int full = total / cus * cus, rest = total - full;
        const bool split = rest > cus / 4 && full > 0 && 2 * rest <= cus;
        p.tiles_n = tn256;
        p.id0 = 0;
        p.count = split ? full : total;
        // the weights widened once into the image (one streaming pass), then loaded straight into LDS by every tile
        const std::size_t img = image_bytes(a.n, a.k);
        // (gemm_pp reads the scales through a buffer descriptor with 32-bit offsets)
        const bool scales32 = a.n * a.ld_s * 4 < (std::size_t{1} << 31);
        if (a.wimage != nullptr && img != 0 && a.wimage_bytes >= img && scales32) {
            p.wimg = static_cast<const unsigned char*>(a.wimage);
            p.wimg_bytes = img;
            p.wsteps = static_cast<int>(a.k / 64);
            if (!a.image_ready) launch_widen(a.w, a.ld_w, a.n, a.k, XT == SEPAL_HIP_F16, a.wimage, stream);
        }
        if (p.wimg != nullptr) {
            // persistent: one block per CU (a multiple of the 8 XCDs)
            const int grid = std::min(p.count, std::max(8, cus / 8 * 8));
            v2::gemm_pp<XT, EP, YT, 4, SPLIT><<<dim3(grid), dim3(512), 0, stream>>>(p);
        }
        else launch_big3<XT, EP, YT, 4, SPLIT>(p, stream);
        if (split) {
            BigParams q = p;
            q.id0 = full;
            q.count = rest;
            if (q.wimg != nullptr) {
                int extra = 0;
                if (a.next_image != nullptr) {
                    // the next multiply's image on blocks dispatched after the halves. When the CUs the halves
                    // leave idle can widen it within the halves' time (measured: ~2.1 us per 128-value group for a
                    // half, ~25 GB/s of image traffic per widening CU), they alone do (the down multiply's halves,
                    // 164 us, against 150 MB); otherwise four blocks per CU, so that every CU joins as its half ends
                    // (the gate/up multiply's halves, ~42 us, against 75 MB: 75 -> 60 us)
                    const int idle = std::max(32, cus - 2 * rest);
                    const double halves_us = 2.1 * static_cast<double>(a.k / 128);
                    const double widen_us = 3.0 * static_cast<double>(a.next_n) * a.next_k / (idle * 25.0e3);
                    extra = widen_us <= halves_us ? idle : 4 * cus;
                    q.jw = reinterpret_cast<const signed char*>(a.next_w);
                    q.j_ld = a.next_ld_w;
                    q.j_n = static_cast<int>(a.next_n);
                    q.j_wsteps = static_cast<int>(a.next_k / 64);
                    q.j_tiles_n = static_cast<int>((a.next_n + 255) / 256);
                    q.j_f16 = a.next_f16;
                    q.j_img = static_cast<unsigned char*>(a.next_image);
                    q.j_blocks = extra;
                    next_done = true;
                }
                v2::gemm_pp<XT, EP, YT, 2, SPLIT><<<dim3(2 * q.count + extra), dim3(512), 0, stream>>>(q);
            } else {
                launch_big3<XT, EP, YT, 2, SPLIT>(q, stream);
            }
        }
    } else if (takes && !wide) {
        // fewer than two rounds of 256 x 256 tiles: the plan's tile height and K split
        p.tiles_n = tn256;
        const SmallGridPlan plan = plan_small_grid(a, tn256, static_cast<int>(a.k / 128), a.config < 0);
        const int lead = plan.rows ? static_cast<int>(a.t / 256) * 256 : 0;
        if (lead > 0) {
            BigParams q = p;
            q.t = lead;
            q.x_bytes = (static_cast<std::size_t>(lead - 1) * a.ld_x + kx) * 2;
            launch_grid<XT, EP, YT, SPLIT>(a, q, 4, 1, false, stream);
        }
        if (lead < static_cast<int>(a.t)) {
            BigParams q = p;
            if (lead > 0) {
                q.t = static_cast<int>(a.t) - lead;
                q.x = p.x + static_cast<std::size_t>(lead) * a.ld_x;
                q.y = static_cast<char*>(p.y) + static_cast<std::size_t>(lead) * y_row_bytes<YT>(a.ld_y);
                q.x_bytes = (static_cast<std::size_t>(q.t - 1) * a.ld_x + kx) * 2;
            }
            if (plan.rows) launch_grid<XT, EP, YT, SPLIT>(a, q, plan.mb2, plan.splits2, plan.planes2, stream);
            else launch_grid<XT, EP, YT, SPLIT>(a, q, plan.mb, plan.splits, plan.planes, stream);
        }
    } else if constexpr (SPLIT == 1 && YT != kYPairs) {
        p.tiles_n = wide ? tn256 : static_cast<int>((a.n + 127) / 128);
        if (wide) launch_big2<XT, EP, YT, 4>(p, stream);
        else launch_big2<XT, EP, YT, 2>(p, stream);
    } else {
        throw LaunchError("gemm_w8g: the hi + lo form (X or Y) runs on the 64-wide-step kernel only");
    }
    check_launch("gemm_w8g large-M kernel launch");
    // the next multiply's image, when no halves launch took it
    if (a.next_image != nullptr && !next_done)
        launch_widen(a.next_w, a.next_ld_w, a.next_n, a.next_k, a.next_f16 != 0, a.next_image, stream);
}

// Whether a problem takes the small-M (weight-streaming) kernels: they write float32 (or SwiGLU outputs); a binary16
// Store always takes the large-M kernels. By default they take T <= 32 with N < 8192: measured on the model's weight
// shapes, the large-M kernels' small-grid plan (64-row blocks, K split) is faster above 32 rows (the streaming kernels
// double their time from 33 rows, at 64-row tiles) and at any T for N >= 8192 (gate/up 19456 x 2560: 20 against
// 24 us at T = 1), and the streaming kernels are faster for the narrow, long-K down shape (2560 x 9728: 22.5 against
// 29 us at T <= 16).
inline bool small_path(const GemmArgs& a) {
    const bool eligible = a.y_type == SEPAL_HIP_F32 || a.epilogue == SEPAL_HIP_SWIGLU;
    return eligible && (a.config == 1 || (a.config < 0 && a.t <= 32 && a.n < 8192));
}

template <int XT, int EP, int YT, int SPLIT>
void dispatch_path(const GemmArgs& a, hipStream_t stream) {
    if constexpr (YT == kYPairs) {
        // only the large-M kernels write the pairs (gemm_w8g_pairs_chain)
        launch_big<XT, EP, YT, SPLIT>(a, stream);
        return;
    }
    if constexpr (SPLIT == 1) {
        // T <= 16 by default: the M <= 16 stack's pass kernels where they take the shape
        SmallGemmPlan plan;
        if (a.config < 0 && a.t <= 16 && small_gemm_plan(a, plan)) {
            launch_small_gemm_w8g(a, plan, stream);
            return;
        }
    }
    if (SPLIT == 1 && small_path(a)) launch_stream_w8g(a, stream);
    else launch_big<XT, EP, YT, SPLIT>(a, stream);
}

template <int XT, int SPLIT>
void dispatch_ep(const GemmArgs& a, hipStream_t stream) {
    switch (a.epilogue) {
    case SEPAL_HIP_STORE:
        if (a.y_type == SEPAL_HIP_F16) dispatch_path<XT, SEPAL_HIP_STORE, SEPAL_HIP_F16, SPLIT>(a, stream);
        else dispatch_path<XT, SEPAL_HIP_STORE, SEPAL_HIP_F32, SPLIT>(a, stream);
        break;
    case SEPAL_HIP_ADD: dispatch_path<XT, SEPAL_HIP_ADD, SEPAL_HIP_F32, SPLIT>(a, stream); break;
    default:
        switch (a.y_type) {
        case SEPAL_HIP_F32: dispatch_path<XT, SEPAL_HIP_SWIGLU, SEPAL_HIP_F32, SPLIT>(a, stream); break;
        case SEPAL_HIP_BF16: dispatch_path<XT, SEPAL_HIP_SWIGLU, SEPAL_HIP_BF16, SPLIT>(a, stream); break;
        case kYPairs:
            if constexpr (XT == SEPAL_HIP_BF16 && SPLIT == 1) dispatch_path<XT, SEPAL_HIP_SWIGLU, kYPairs, SPLIT>(a, stream);
            else throw LaunchError("gemm_w8g: hi + lo pair output needs a bf16 X");
            break;
        default: dispatch_path<XT, SEPAL_HIP_SWIGLU, SEPAL_HIP_F16, SPLIT>(a, stream); break;
        }
    }
}

// ---- float32 X: the hi + lo split ----------------------------------------------------------------------------------
//
// A float32 x is the sum of hi = bf16(x) (nearest even) and lo = bf16(x - hi); x - hi is exact in float32 and lo is
// within 2^-9 of it, so hi + lo is within 2^-17 |x| of x. Each bf16 times an int8 weight is exact in the float32
// accumulator, so the multiply of the pair is the float32 product within that bound plus the accumulation's rounding.

// x float32 [t, ld_x] -> pairs. Layout 0 (for gemm_big3's hi + lo form): one row of 2k bf16 per token, the 64-value
// chunk j of k stored as chunk 2j (hi) and 2j + 1 (lo). Layout 1: hi [t, k] at out, lo [t, k] at out + t k.
__global__ void __launch_bounds__(256) split_kernel(const float* __restrict__ x, std::size_t ld_x, unsigned short* __restrict__ out,
                                                    int t, int k, int layout) {
    const int per_row = k / 8;
    const std::size_t total = static_cast<std::size_t>(t) * per_row;
    for (std::size_t id = blockIdx.x * 256ull + threadIdx.x; id < total; id += static_cast<std::size_t>(gridDim.x) * 256) {
        const int r = static_cast<int>(id / per_row), k0 = 8 * static_cast<int>(id % per_row);
        const float* src = x + static_cast<std::size_t>(r) * ld_x + k0;
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(src), v1 = *reinterpret_cast<const f32x4*>(src + 4);
        unsigned hi[4], lo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = i < 2 ? v0[2 * i] : v1[2 * i - 4], b = i < 2 ? v0[2 * i + 1] : v1[2 * i - 3];
            const unsigned short ha = f32_to_bf16_bits(a), hb = f32_to_bf16_bits(b);
            const unsigned short la = f32_to_bf16_bits(__fsub_rn(a, bf16_bits_to_f32(ha)));
            const unsigned short lb = f32_to_bf16_bits(__fsub_rn(b, bf16_bits_to_f32(hb)));
            hi[i] = ha | (static_cast<unsigned>(hb) << 16);
            lo[i] = la | (static_cast<unsigned>(lb) << 16);
        }
        unsigned short *dh, *dl;
        if (layout == 0) {
            dh = out + static_cast<std::size_t>(r) * (2 * k) + 128 * (k0 / 64) + k0 % 64;
            dl = dh + 64;
        } else {
            dh = out + static_cast<std::size_t>(r) * k + k0;
            dl = dh + static_cast<std::size_t>(t) * k;
        }
        *reinterpret_cast<u32x4*>(dh) = u32x4{hi[0], hi[1], hi[2], hi[3]};
        *reinterpret_cast<u32x4*>(dl) = u32x4{lo[0], lo[1], lo[2], lo[3]};
    }
}

// y[t, f] = swiglu(z[t, 128 (f / 64) + f % 64], z[t, 128 (f / 64) + 64 + f % 64]) for the f < n / 2 outputs.
template <int YT>
__global__ void __launch_bounds__(256) swiglu_rows_kernel(const float* __restrict__ z, int n, void* __restrict__ y,
                                                          std::size_t ld_y, int t) {
    const int half = n / 2;
    const std::size_t total = static_cast<std::size_t>(t) * half;
    for (std::size_t id = blockIdx.x * 256ull + threadIdx.x; id < total; id += static_cast<std::size_t>(gridDim.x) * 256) {
        const int r = static_cast<int>(id / half), f = static_cast<int>(id % half);
        const float* zr = z + static_cast<std::size_t>(r) * n + 128 * (f / 64) + f % 64;
        store_out<YT>(y, static_cast<std::size_t>(r) * ld_y + f, swiglu_libm(zr[0], zr[64]));
    }
}

inline int grid_for(std::size_t items) {
    return static_cast<int>(std::min<std::size_t>((items + 255) / 256, std::size_t{8192}));
}

void launch_f32(const GemmArgs& a, hipStream_t stream) {
    if (a.xsplit == nullptr) throw LaunchError("gemm_w8g: float32 X needs the split buffer");
    const int t = static_cast<int>(a.t), k = static_cast<int>(a.k);
    auto* pairs = static_cast<unsigned short*>(a.xsplit);
    if (!small_path(a) && big3_takes(a, 2 * a.k, 2 * a.k)) {
        // one pass of the 64-wide-step kernel over the hi + lo row (twice the MFMAs of a 16-bit X)
        split_kernel<<<grid_for(a.t * (a.k / 8)), 256, 0, stream>>>(static_cast<const float*>(a.x), a.ld_x, pairs, t, k, 0);
        check_launch("gemm_w8g split launch");
        GemmArgs b = a;
        b.x = pairs;
        b.x_type = SEPAL_HIP_BF16;
        b.ld_x = 2 * a.k;
        dispatch_ep<SEPAL_HIP_BF16, 2>(b, stream);
        return;
    }
    // any other path: hi and lo as two bf16 multiplies, the second added in float32
    split_kernel<<<grid_for(a.t * (a.k / 8)), 256, 0, stream>>>(static_cast<const float*>(a.x), a.ld_x, pairs, t, k, 1);
    check_launch("gemm_w8g split launch");
    GemmArgs hi = a, lo = a;
    hi.x = pairs;
    lo.x = pairs + a.t * a.k;
    hi.x_type = lo.x_type = SEPAL_HIP_BF16;
    hi.ld_x = lo.ld_x = a.k;
    lo.epilogue = SEPAL_HIP_ADD;
    if (a.epilogue == SEPAL_HIP_SWIGLU) {
        if (a.ytmp == nullptr) throw LaunchError("gemm_w8g: float32 X with SwiGLU needs the sum buffer");
        hi.y = lo.y = a.ytmp;
        hi.y_type = lo.y_type = SEPAL_HIP_F32;
        hi.ld_y = lo.ld_y = a.n;
        hi.epilogue = SEPAL_HIP_STORE;
    }
    dispatch_ep<SEPAL_HIP_BF16, 1>(hi, stream);
    dispatch_ep<SEPAL_HIP_BF16, 1>(lo, stream);
    if (a.epilogue == SEPAL_HIP_SWIGLU) {
        const int g = grid_for(a.t * (a.n / 2));
        const int n = static_cast<int>(a.n);
        if (a.y_type == SEPAL_HIP_F32) swiglu_rows_kernel<SEPAL_HIP_F32><<<g, 256, 0, stream>>>(a.ytmp, n, a.y, a.ld_y, t);
        else if (a.y_type == SEPAL_HIP_BF16) swiglu_rows_kernel<SEPAL_HIP_BF16><<<g, 256, 0, stream>>>(a.ytmp, n, a.y, a.ld_y, t);
        else swiglu_rows_kernel<SEPAL_HIP_F16><<<g, 256, 0, stream>>>(a.ytmp, n, a.y, a.ld_y, t);
        check_launch("gemm_w8g swiglu launch");
    }
}

} // namespace w8g

bool gemm_w8g_pairs_chain(const GemmArgs& gu, const GemmArgs& dn) {
    GemmArgs d = dn;
    d.x_type = SEPAL_HIP_F32;
    d.y_type = SEPAL_HIP_F32;
    GemmArgs g = gu;
    g.y_type = SEPAL_HIP_F32;
    return gu.epilogue == SEPAL_HIP_SWIGLU && gu.x_type == SEPAL_HIP_BF16 && gu.t > kSmallM && !w8g::small_path(g) &&
           w8g::big3_takes(g, g.k, g.ld_x) && dn.k == gu.n / 2 && !w8g::small_path(d) && w8g::big3_takes(d, 2 * d.k, 2 * d.k);
}

void launch_gemm_w8g_pairs(const GemmArgs& dn, hipStream_t stream) {
    GemmArgs b = dn;
    b.x_type = SEPAL_HIP_BF16;
    w8g::dispatch_ep<SEPAL_HIP_BF16, 2>(b, stream);
}

void launch_gemm_w8g(const GemmArgs& a, hipStream_t stream) {
    if (a.x_type == SEPAL_HIP_F32) w8g::launch_f32(a, stream);
    else if (a.x_type == SEPAL_HIP_BF16) w8g::dispatch_ep<SEPAL_HIP_BF16, 1>(a, stream);
    else w8g::dispatch_ep<SEPAL_HIP_F16, 1>(a, stream);
}

std::size_t gemm_w8g_image_bytes(const GemmArgs& a) {
    if (a.t <= kSmallM) return 0;
    const std::size_t tiles = (a.t + 255) / 256 * ((a.n + 255) / 256);
    if (tiles < 2 * 256 || (a.epilogue == SEPAL_HIP_SWIGLU && a.n % 256 != 0)) return 0;
    return w8g::image_bytes(a.n, a.k);
}

std::size_t w8g_image_bytes_nk(std::size_t n, std::size_t k) { return k % 64 == 0 ? w8g::image_bytes(n, k) : 0; }

void launch_w8g_image(const std::int8_t* w, std::size_t ld_w, std::size_t n, std::size_t k, bool f16, void* img,
                      hipStream_t stream) {
    w8g::launch_widen(w, ld_w, n, k, f16, img, stream);
}

std::size_t gemm_w8g_scratch_bytes(const GemmArgs& a) {
    if (a.x_type != SEPAL_HIP_F32) return 0;
    const auto up256 = [](std::size_t b) { return (b + 255) / 256 * 256; };
    const bool one_pass = !w8g::small_path(a) && w8g::big3_takes(a, 2 * a.k, 2 * a.k);
    return up256(a.t * a.k * 4) + (!one_pass && a.epilogue == SEPAL_HIP_SWIGLU ? up256(a.t * a.n * 4) : 0);
}

} // namespace sepal::hip

