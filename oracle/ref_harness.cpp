// C entry points over the reference's own CPU int8 GEMM (compiled from the reference sources by oracle/Makefile into
// oracle/_ref/). Test infrastructure only: used to write the golden fixtures under tests/golden/, to pin the C oracle,
// and as bench.py's CPU baseline ("kind": "reference"). It calls the reference API as the reference's own tests do
// (runner/tests/test_cpu_gemm.cpp:70-80 run_gemm) and unpacks the packed panels back to row-major arrays using the
// panel layout documented in runner/include/sepal/cpu/gemm.hpp:52-100 and runner/src/cpu/gemm.cpp:116-165.
#include <algorithm>
#include <chrono>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>
#include <vector>

#include "sepal/cpu/elementwise.hpp"
#include "sepal/cpu/gemm.hpp"
#include "sepal/cpu/isa.hpp"
#include "sepal/cpu/thread_pool.hpp"

using namespace sepal::cpu;

namespace {

thread_local std::string g_error;

template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return 1;
    }
}

Isa pick_isa() { return best_isa(); }

} // namespace

extern "C" {

const char* ref_last_error() { return g_error.c_str(); }

// 1 when the reference picks its I8_Z (AVX-512 VNNI, 128-blocks) kernel on this CPU, 0 for I8_Y.
int ref_i8_variant_is_z() { return pick_variant(WeightKind::I8, pick_isa()) == Variant::I8_Z ? 1 : 0; }

unsigned ref_default_threads() { return default_thread_count(); }

// pack_weight(I8): q [n][k] int8, scale [n][kblocks], corr [n][kblocks] (row-major, unpacked from the panels).
int ref_pack_weight_i8(const float* w, std::size_t n, std::size_t k, std::int8_t* q, float* scale, std::int32_t* corr) {
    return guarded([&] {
        ThreadPool pool(1);
        const PackedWeight pw = pack_weight(w, k, n, k, WeightKind::I8, pick_isa(), pool);
        if (pw.variant() != Variant::I8_Z) throw std::runtime_error("the reference picked I8_Y on this CPU");
        const std::size_t nr = 32, g = 4, kb = pw.kblocks();
        for (std::size_t c = 0; c < n; ++c) {
            const std::size_t p = c / nr, jj = c % nr;
            const auto* panel = reinterpret_cast<const std::int8_t*>(pw.panel(p));
            for (std::size_t kk = 0; kk < k; ++kk) q[c * k + kk] = panel[((kk / g) * nr + jj) * g + kk % g];
            for (std::size_t b = 0; b < kb; ++b) {
                scale[c * kb + b] = pw.scale(p)[b * nr + jj];
                corr[c * kb + b] = pw.corr(p)[b * nr + jj];
            }
        }
    });
}

// pack_acts(I8_Z): q [rows][k] int8 (the stored u8 minus 128), scale [rows][kblocks].
int ref_pack_acts_i8(const float* x, std::size_t rows, std::size_t k, std::int8_t* q, float* scale) {
    return guarded([&] {
        ThreadPool pool(1);
        PackedActs pa;
        pack_acts(pa, x, k, rows, k, Variant::I8_Z, pool);
        const std::size_t mr = 12, g = 4, kb = pa.kblocks;
        for (std::size_t r = 0; r < rows; ++r) {
            const std::size_t mb = r / mr, rr = r % mr;
            const unsigned char* blk = pa.data.data() + mb * pa.block_bytes;
            for (std::size_t kk = 0; kk < k; ++kk)
                q[r * k + kk] = static_cast<std::int8_t>(static_cast<int>(blk[((kk / g) * mr + rr) * g + kk % g]) - 128);
            for (std::size_t b = 0; b < kb; ++b) scale[r * kb + b] = pa.row_scale[(mb * kb + b) * mr + rr];
        }
    });
}

// y [rows][n] = (accumulate ? y : 0) + the reference cpu-q8 product of x [rows][k] and w [n][k].
int ref_gemm_i8(const float* x, std::size_t rows, const float* w, std::size_t n, std::size_t k, float* y, int accumulate,
                unsigned threads) {
    return guarded([&] {
        ThreadPool pool(threads);
        const PackedWeight pw = pack_weight(w, k, n, k, WeightKind::I8, pick_isa(), pool);
        PackedActs pa;
        pack_acts(pa, x, k, rows, k, pw.variant(), pool);
        gemm_packed(pw, pa, y, n, accumulate != 0, pool);
    });
}

// y [rows][n] = silu(x gate^T) * (x up^T) by the reference cpu-q8 SwiGLU product (gate, up [n][k]).
int ref_gemm_i8_swiglu(const float* x, std::size_t rows, const float* gate, const float* up, std::size_t n, std::size_t k,
                       float* y, unsigned threads) {
    return guarded([&] {
        ThreadPool pool(threads);
        const PackedWeight pw = pack_weight_swiglu(gate, up, k, n, k, WeightKind::I8, pick_isa(), pool);
        PackedActs pa;
        pack_acts(pa, x, k, rows, k, pw.variant(), pool);
        gemm_packed(pw, pa, y, n, false, pool);
    });
}

// The reference's AVX2 int8 path, Variant::I8_Y (kernel_i8_y, runner/src/cpu/gemm_kernels_avx2.cpp:40-79): one
// activation scale per row and one weight scale per feature (a single block spanning k), int16 pairs of int8 values,
// forced by packing for Isa::Avx2 (runner/src/cpu/gemm.cpp:58-62). y [rows][n] = (accumulate ? y : 0) + product.
int ref_gemm_i8y(const float* x, std::size_t rows, const float* w, std::size_t n, std::size_t k, float* y, int accumulate,
                 unsigned threads) {
    return guarded([&] {
        ThreadPool pool(threads);
        const PackedWeight pw = pack_weight(w, k, n, k, WeightKind::I8, Isa::Avx2, pool);
        if (pw.variant() != Variant::I8_Y) throw std::runtime_error("the reference did not pick I8_Y for Isa::Avx2");
        PackedActs pa;
        pack_acts(pa, x, k, rows, k, pw.variant(), pool);
        gemm_packed(pw, pa, y, n, accumulate != 0, pool);
    });
}

// The I8_Y SwiGLU product (pack_weight_swiglu for Isa::Avx2): y [rows][n] = silu(x gate^T) * (x up^T).
int ref_gemm_i8y_swiglu(const float* x, std::size_t rows, const float* gate, const float* up, std::size_t n, std::size_t k,
                        float* y, unsigned threads) {
    return guarded([&] {
        ThreadPool pool(threads);
        const PackedWeight pw = pack_weight_swiglu(gate, up, k, n, k, WeightKind::I8, Isa::Avx2, pool);
        if (pw.variant() != Variant::I8_Y) throw std::runtime_error("the reference did not pick I8_Y for Isa::Avx2");
        PackedActs pa;
        pack_acts(pa, x, k, rows, k, pw.variant(), pool);
        gemm_packed(pw, pa, y, n, false, pool);
    });
}

// pack_weight(I8, Isa::Avx2): q [n][k] int8 (from the int16 pairs) and one scale per feature, unpacked from the panels
// (nr 16, group 2: value kk of column jj at ((kk / 2) * 16 + jj) * 2 + kk % 2, runner/src/cpu/gemm.cpp:137-165).
int ref_pack_weight_i8y(const float* w, std::size_t n, std::size_t k, std::int8_t* q, float* scale) {
    return guarded([&] {
        ThreadPool pool(1);
        const PackedWeight pw = pack_weight(w, k, n, k, WeightKind::I8, Isa::Avx2, pool);
        if (pw.variant() != Variant::I8_Y) throw std::runtime_error("the reference did not pick I8_Y for Isa::Avx2");
        const std::size_t nr = 16, g = 2;
        for (std::size_t c = 0; c < n; ++c) {
            const std::size_t p = c / nr, jj = c % nr;
            const auto* panel = reinterpret_cast<const std::int16_t*>(pw.panel(p));
            for (std::size_t kk = 0; kk < k; ++kk) q[c * k + kk] = static_cast<std::int8_t>(panel[((kk / g) * nr + jj) * g + kk % g]);
            scale[c] = pw.scale(p)[jj];
        }
    });
}

int ref_rmsnorm(const float* x, std::size_t rows, std::size_t cols, const float* w1, double eps, float* y) {
    return guarded([&] {
        ThreadPool pool(1);
        rmsnorm_rows(x, cols, y, cols, rows, cols, w1, eps, pool);
    });
}

// Timing of one cpu-q8 MLP block as the reference runs it (runner/src/cpu/trunk.cpp:286-298): weights packed once,
// then per call pack_acts(x) -> gemm_packed(gate_up, SwiGLU) -> pack_acts(h) -> gemm_packed(down). Returns the median
// seconds of `reps` timed calls after one warm-up, and the median seconds spent in pack_acts alone (pack_s).
int ref_time_mlp_block(const float* x, std::size_t rows, const float* gate, const float* up, const float* down,
                       std::size_t hidden, std::size_t inter, unsigned threads, int reps, double* total_s,
                       double* pack_s, unsigned* threads_used) {
    return guarded([&] {
        ThreadPool pool(threads);
        *threads_used = pool.size();
        const PackedWeight gu = pack_weight_swiglu(gate, up, hidden, inter, hidden, WeightKind::I8, pick_isa(), pool);
        const PackedWeight dn = pack_weight(down, inter, hidden, inter, WeightKind::I8, pick_isa(), pool);
        std::vector<float> h(rows * inter), y(rows * hidden);
        PackedActs pa, ph;
        std::vector<double> totals, packs;
        for (int r = 0; r <= reps; ++r) {
            const auto t0 = std::chrono::steady_clock::now();
            pack_acts(pa, x, hidden, rows, hidden, gu.variant(), pool);
            const auto t1 = std::chrono::steady_clock::now();
            gemm_packed(gu, pa, h.data(), inter, false, pool);
            const auto t2 = std::chrono::steady_clock::now();
            pack_acts(ph, h.data(), inter, rows, inter, dn.variant(), pool);
            const auto t3 = std::chrono::steady_clock::now();
            gemm_packed(dn, ph, y.data(), hidden, false, pool);
            const auto t4 = std::chrono::steady_clock::now();
            if (r == 0) continue;
            totals.push_back(std::chrono::duration<double>(t4 - t0).count());
            packs.push_back(std::chrono::duration<double>((t1 - t0) + (t3 - t2)).count());
        }
        std::sort(totals.begin(), totals.end());
        std::sort(packs.begin(), packs.end());
        *total_s = totals[totals.size() / 2];
        *pack_s = packs[packs.size() / 2];
    });
}

} // extern "C"
