/*
 * CPU oracle of the W8g128 quantized-MLP path: a plain-C restatement of the reference's algorithms, used ONLY as the
 * checker (tests/, __graft_entry__.smoke(), bench.py's cpu_baseline leg). Nothing in the product path links it.
 *
 * Every function names the reference file:line whose behaviour it restates (paths relative to the reference root,
 * bloomifycafe/Sepal-Runner). All matrices are row-major with explicit row strides counted in elements.
 *
 * Pinning (what each function is checked against, see tests/test_oracle.py):
 *   orc_quantize_group_r1   closed form of the reference's host copy + special cases (zero group, outlier, +-127,
 *                           half-step error bound); the reference CUDA packer cannot be built here.
 *   orc_quantize_block_r2   bit-exact against golden fixtures dumped from the compiled reference CPU library
 *                           (pack_weight / pack_acts, I8_Z), plus the same special cases.
 *   orc_group_sums          brute-force int64 sums on tiny shapes; the integer identity corr = 128 * sum(q).
 *   orc_gemm_q8             bit-exact against the compiled reference gemm_packed (I8_Z) fixtures: Store, Add, SwiGLU.
 *   orc_gemm_q8y            bit-exact against the compiled reference gemm_packed (I8_Y, the AVX2 kernel forced by
 *                           packing for Isa::Avx2) fixtures: Store, Add, SwiGLU.
 *   orc_gemm_w8g            float64 brute force bound and the group identity sum_g s_g * sum_k x q; the fmaf chain
 *                           order is the reference's stated schedule (CUDA source, not buildable here).
 *   orc_exp_cephes / silu   bit-exact via orc_gemm_q8's SwiGLU fixtures; against libm exp within 2 ulp.
 *   orc_swiglu_libm         "parity unpinned" at the ulp level: the reference GPU path calls CUDA expf/log1pf; pinned by
 *                           tolerance against float64 silu(g)*u only.
 *   orc_rmsnorm_rows        bit-exact against the compiled reference rmsnorm_rows fixtures.
 *   orc_s8_quantize_rows    the rule's closed-form cases: zero rows (scale 0, q 0), the row maximum at +-127, ties
 *                           rounded to even where 127 / amax is exactly 1, the half-step bound, smoothing as a
 *                           pre-multiplied input (the reference CUDA quantizer cannot be built here).
 *   orc_gemm_s8             the integer sum against numpy int64 products; the float32 order by hand-checked cases.
 */
#ifndef SEPAL_ORACLE_H
#define SEPAL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_STORE = 0, ORC_ADD = 1, ORC_SWIGLU = 2 };

/* bfloat16 <-> float32, round to nearest even, NaN kept quiet (runner/src/cpu/gemm.cpp:73-78). */
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t b);

/* Packed gate/up row order of the fused SwiGLU multiply: packed row p comes from source row
 * orc_gate_up_source(p, inter), gate rows 0..inter-1, up rows inter..2*inter-1
 * (runner/cuda/src/gemm_simt_kernels.hpp:72-77). */
size_t orc_gate_up_source(size_t p, size_t inter);

/* R1 "divide" group quantizer of the gpu-w8g load-time packer: per (row, 128-group) m = max|w|, s = m / 127,
 * q = clamp(rint(w / s), -127, 127), an all-zero group gets s = 0 and q = 0.
 * (runner/cuda/src/gemm_simt_kernels.cu:266-286; host copy runner/cuda/tests/test_gemm_simt_kernels.cpp:71-89.) */
void orc_quantize_group_r1(const float* src, size_t ld_src, size_t rows, size_t k, int8_t* q, size_t ld_q, float* s,
                           size_t ld_s);

/* R2 "reciprocal-multiply" quantizer of cpu-q8 (weights and activations alike): per (row, block) amax = max|x|,
 * s = amax > 0 ? amax / 127 : 1, q = clamp(nearbyint(x * (1 / s)), -127, 127). The last block may be short.
 * `block` is 128 for I8_Z, or k for one scale per row.
 * (runner/src/cpu/gemm.cpp:103-106 quantise, :137-164 weights, :285-306 activations.) */
void orc_quantize_block_r2(const float* src, size_t ld_src, size_t rows, size_t k, size_t block, int8_t* q, size_t ld_q,
                           float* s, size_t ld_s);

/* Exact int32 per-(128-group) sums S[g][t][n] = sum_{k in g} xq[t,k] * wq[n,k]
 * (runner/src/cpu/gemm_kernels_avx512.cpp:82-93: vpdpbusd with the -corr start is this sum exactly). */
void orc_group_sums(const int8_t* xq, size_t ld_xq, const int8_t* wq, size_t ld_wq, size_t t, size_t n, size_t k,
                    int32_t* sums);

/* cpu-q8 I8_Z multiply. For each output: f_b = float(S_b) over weight blocks of 128.
 * act_block = 128 (the reference I8_Z): y = f_0 * (ws_0 * xs[t,0]), then y = fma(f_b, ws_b * xs[t,b], y), b = 1, 2, ...
 * act_block = k > 128 (one activation scale per token, BASELINE's gpu-q8w wording; the reference has no multiply with
 * per-token activation scales and per-group weight scales, so this chain is this repository's definition):
 * y = (f_0 * ws_0, then fma(f_b, ws_b, y)) * xs[t,0].
 * Epilogue: Store; Add (y_out = y_out + y); SwiGLU on 64-row interleaved gate/up weights [2I, K] (orc_gate_up_source),
 * Y[t, 64c + r] = silu_cephes(acc[128c + r]) * acc[128c + 64 + r] with n = 2I.
 * (runner/src/cpu/gemm_kernels_avx512.cpp:74 Z_FLUSH_I, :102-113; runner/src/cpu/gemm.cpp:417-447 finish_tile;
 *  emulation in runner/tests/test_cpu_gemm.cpp:194-203.) */
/* kernel_i8_y (runner/src/cpu/gemm_kernels_avx2.cpp:40-79): one activation scale per row, one weight scale per
 * feature; y = (float(S) * ws[n]) * xs[t], S the exact int32 sum over k; finish_tile epilogues as orc_gemm_q8. */
void orc_gemm_q8y(const int8_t* xq, size_t ld_xq, const float* xs, const int8_t* wq, size_t ld_wq, const float* ws,
                  float* y, size_t ld_y, size_t t, size_t n, size_t k, int epilogue);
void orc_gemm_q8(const int8_t* xq, size_t ld_xq, const float* xs, size_t ld_xs, size_t act_block, const int8_t* wq,
                 size_t ld_wq, const float* ws, size_t ld_ws, float* y, size_t ld_y, size_t t, size_t n, size_t k,
                 int epilogue);

/* Cephes-style exp with the reference's clamps and degree-5 polynomial, one lane (runner/src/cpu/vmath.hpp:16-32),
 * and silu(x) = x / (1 + exp(-x)) (vmath.hpp:35-38). */
float orc_exp_cephes(float x);
float orc_silu_cephes(float x);

/* gpu-w8g multiply: per output acc = fmaf(x[t,k], fl(q[n,k] * s[n,k/128]), acc) for k = 0..K-1 from 0, then the
 * epilogue; SwiGLU as orc_gemm_q8 but with orc_swiglu_libm.
 * (runner/cuda/src/gemm_simt_kernels.cu:172-178 dequantise, :197-200 chain, :206-239 epilogues;
 *  emulation runner/cuda/tests/test_gemm_simt_kernels.cpp:152-157.) */
void orc_gemm_w8g(const float* x, size_t ld_x, const int8_t* q, size_t ld_q, const float* s, size_t ld_s, float* y,
                  size_t ld_y, size_t t, size_t n, size_t k, int epilogue);

/* silu(g) * u as the reference GPU computes it: fl(fl(g * exp(-softplus(-g))) * u), softplus(x) = max(x,0) +
 * log1p(exp(-|x|)) with the C library's expf / log1pf (runner/cuda/src/gemm_simt_kernels.cu:27-29). */
float orc_swiglu_libm(float g, float u);

/* RMSNorm of rows: sum of squares in the reference's fixed order (four 8-lane fma accumulators over chunks of 32, a
 * tail of 8-chunks into the first, then (a0+a1)+(a2+a3) and the pairwise lane sum), mean in double,
 * inv = (float)(1 / sqrt(mean + eps)), y = (x * inv) * w1 (w1 NULL means ones). cols a multiple of 8.
 * (runner/src/cpu/elementwise.cpp:22-39 sum_squares, :43-59 rmsnorm_rows; vmath.hpp:52-59 hsum_ps.) */
void orc_rmsnorm_rows(const float* x, size_t ld_x, float* y, size_t ld_y, size_t rows, size_t cols, const float* w1,
                      double eps);

/* The GPU int8 path's per-row quantizer (launch_quantize_rows_s8, and launch_quantize_weights_s8's Plain layout): per
 * row v = x * smooth[c] in float32 (smooth NULL: x), amax = max |v|, inv = amax > 0 ? 127 / amax : 0, scale =
 * amax / 127, q = clamp(rint(v * inv), -127, 127).
 * (runner/cuda/src/gemm_s8_kernels.cu:29-32 quantize_one, :50-79 rows, :82-110 weights; host form
 *  runner/cuda/tests/test_gemm_s8_kernels.cpp:58-68.) */
void orc_s8_quantize_rows(const float* x, size_t ld_x, const float* smooth, size_t rows, size_t cols, int8_t* q, size_t ld_q,
                          float* scales);

/* The int8-activation multiply with per-channel scales: S = exact integer sum over k of xq[t,k] * wq[n,k] (int32),
 * y = ((float)S * sx[t]) * sw[n] in float32 (runner/cuda/src/gemm_s8_kernels.cu:255-266; closed form
 * runner/cuda/tests/test_gemm_s8_kernels.cpp:208-213). */
void orc_gemm_s8(const int8_t* xq, size_t ld_x, const float* sx, const int8_t* wq, size_t ld_w, const float* sw, float* y,
                 size_t ld_y, size_t t, size_t n, size_t k);

#ifdef __cplusplus
}
#endif

#endif
