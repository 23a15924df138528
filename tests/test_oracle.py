"""The CPU oracle pinned before it is trusted (CPU only).

Pins: (1) bit-exact against the golden fixtures dumped from the reference's own compiled CPU code (the reference
test suite's shapes and LCG inputs, MLP-shaped cases, RMSNorm); (2) closed forms and special cases of the quantizers
(zero group, outlier, +-127, half-step bound, the R1/R2 difference on real data); (3) brute force integer sums and the
float64 product for the w8g chain; (4) the exp polynomial against libm.
"""
import numpy as np
import pytest

from oracle import orc
from helpers import max_rel_over_rms, same_bits


def test_r2_quantizer_matches_reference_pack(golden):
    g = golden["ref_suite"]
    for i in range(int(g["count"])):
        w, x = g[f"c{i}_w"], g[f"c{i}_x"]
        q, s = orc.quantize_block_r2(w)
        assert same_bits(q, g[f"c{i}_wq"]) and same_bits(s, g[f"c{i}_ws"])
        kb = s.shape[1]
        k = w.shape[1]
        # corr = 128 * sum of the block's quantized weights (runner/src/cpu/gemm.cpp:163)
        sums = np.stack([q[:, b * 128:min(k, (b + 1) * 128)].astype(np.int64).sum(1) for b in range(kb)], 1)
        assert np.array_equal(128 * sums, g[f"c{i}_corr"])
        xq, xs = orc.quantize_block_r2(x)
        assert same_bits(xq, g[f"c{i}_xq"]) and same_bits(xs, g[f"c{i}_xs"])


def test_q8_chain_matches_reference_gemm(golden):
    g = golden["ref_suite"]
    for i in range(int(g["count"])):
        xq, xs = orc.quantize_block_r2(g[f"c{i}_x"])
        wq, ws = orc.quantize_block_r2(g[f"c{i}_w"])
        assert same_bits(orc.gemm_q8(xq, xs, wq, ws), g[f"c{i}_y"])
        assert same_bits(orc.gemm_q8(xq, xs, wq, ws, epilogue=orc.ADD, y=g[f"c{i}_y_base"]), g[f"c{i}_y_acc"])


def test_q8_mlp_cases_match_reference(golden):
    g = golden["ref_mlp"]
    for i in range(int(g["count"])):
        x = g[f"c{i}_x"]
        xq, xs = orc.quantize_block_r2(x)
        wq, ws = orc.quantize_block_r2(g[f"c{i}_w"])
        assert same_bits(orc.gemm_q8(xq, xs, wq, ws), g[f"c{i}_y"])
        assert same_bits(orc.gemm_q8(xq, xs, wq, ws, epilogue=orc.ADD, y=g[f"c{i}_base"]), g[f"c{i}_y_acc"])
        W = orc.interleave_gate_up(g[f"c{i}_gate"], g[f"c{i}_up"])
        Wq, Ws = orc.quantize_block_r2(W)
        assert same_bits(orc.gemm_q8(xq, xs, Wq, Ws, epilogue=orc.SWIGLU), g[f"c{i}_y_swiglu"])


def test_rmsnorm_matches_reference(golden):
    g = golden["ref_rmsnorm"]
    for i in range(3):
        assert same_bits(orc.rmsnorm_rows(g[f"x{i}"]), g[f"y{i}"])


def test_group_sums_brute_force():
    rng = np.random.default_rng(1)
    xq = rng.integers(-127, 128, size=(7, 384), dtype=np.int8)
    wq = rng.integers(-127, 128, size=(5, 384), dtype=np.int8)
    sums = orc.group_sums(xq, wq)
    for gi in range(3):
        ref = xq[:, gi * 128:(gi + 1) * 128].astype(np.int64) @ wq[:, gi * 128:(gi + 1) * 128].astype(np.int64).T
        assert np.array_equal(sums[gi], ref)
    # extremes: 128 products of -127 * -127 = 2,064,512 per group, exact in int32 and in float32
    xq[:] = -127
    wq[:] = -127
    assert np.all(orc.group_sums(xq, wq) == 128 * 127 * 127)


def test_q8_per_token_chain_closed_form():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((6, 384)).astype(np.float32)
    w = (rng.standard_normal((32, 384)) * 0.02).astype(np.float32)
    xq, xs = orc.quantize_block_r2(x, block=384)
    wq, ws = orc.quantize_block_r2(w)
    y = orc.gemm_q8(xq, xs, wq, ws, act_block=384)
    S = orc.group_sums(xq, wq).astype(np.float32)  # [g, t, n]
    ref = np.zeros((6, 32), np.float32)
    for t in range(6):
        for n in range(32):
            acc = np.float32(S[0, t, n] * ws[n, 0])
            for b in range(1, 3):
                acc = np.float32(np.float64(S[b, t, n]) * np.float64(ws[n, b]) + np.float64(acc))  # exact fma in f64
            ref[t, n] = np.float32(acc * xs[t, 0])
    assert same_bits(y, ref)


def test_r1_quantizer_closed_form_and_special_cases():
    # the reference's simt_quant case (runner/cuda/tests/test_gemm_simt_kernels.cpp:275-302)
    rng = np.random.default_rng(53)
    rows, k = 37, 640
    w = (rng.uniform(-1, 1, (rows, k)) * 0.05).astype(np.float32)
    w[5, 256:384] = 0.0
    w[0, 7] = 3.0
    q, s = orc.quantize_group_r1(w)
    assert s[5, 2] == 0.0 and not q[5, 256:384].any()
    m = np.abs(w.reshape(rows, k // 128, 128)).max(-1)
    assert same_bits(s, (m / np.float32(127.0)).astype(np.float32))
    # closed form: rint(w / s) with a correctly rounded float32 division
    ss = np.repeat(s, 128, axis=1)
    with np.errstate(divide="ignore", invalid="ignore"):
        ref = np.where(ss > 0, np.clip(np.rint((w / ss).astype(np.float32)), -127, 127), 0).astype(np.int8)
    assert np.array_equal(q, ref)
    assert q[0, 7] == 127 and np.abs(q).max() == 127
    step = ss.astype(np.float64)
    err = np.abs(q.astype(np.float64) * step - w) / np.where(step > 0, step, 1)
    assert err.max() <= 0.5 + 1e-6


def test_s8_row_quantizer_rule():
    """The GPU int8 path's rule (127 / amax, zero rows scale 0), by its closed-form cases: where 127 / amax is exactly
    1 the values round half to even; the row maximum maps to +-127; a zero row gets scale 0 and zeros; every value is
    within half a step; the smoothing factor acts as a pre-multiplied input; a plausible mix-up with the cpu-q8 rule
    (1 / (amax / 127), scale 1 on zero rows) differs on the zero row's scale and on real data."""
    x = np.array([[0, 0, 0, 0], [127, 2.5, 3.5, -2.5], [-127, 0.5, 1.5, -0.5]], np.float32)
    q, s = orc.s8_quantize_rows(x)
    assert q[0].tolist() == [0, 0, 0, 0] and s[0] == 0.0
    assert q[1].tolist() == [127, 2, 4, -2] and s[1] == 1.0
    assert q[2].tolist() == [-127, 0, 2, 0] and s[2] == 1.0
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 512)) * rng.uniform(0.01, 30, (64, 1))).astype(np.float32)
    x[5] = 0.0
    q, s = orc.s8_quantize_rows(x)
    amax = np.abs(x).max(1)
    assert np.array_equal(np.abs(q).max(1)[amax > 0], np.full((amax > 0).sum(), 127))
    assert s[5] == 0.0 and not q[5].any()
    assert np.all(np.abs(q.astype(np.float64) * s[:, None] - x) <= s[:, None] * (0.5 + 1e-5) + 1e-30)
    sm = rng.uniform(0.5, 2.0, 512).astype(np.float32)
    q2, s2 = orc.s8_quantize_rows(x, smooth=sm)
    q3, s3 = orc.s8_quantize_rows((x * sm).astype(np.float32))
    assert same_bits(q2, q3) and same_bits(s2, s3)
    qr, sr = orc.quantize_block_r2(x, block=512)
    assert sr[5, 0] == 1.0
    xh = rng.standard_normal((512, 2048)).astype(np.float16).astype(np.float32)
    assert (orc.s8_quantize_rows(xh)[0] != orc.quantize_block_r2(xh, block=2048)[0]).any()  # 127 / amax vs 1 / (amax / 127)


def test_gemm_s8_closed_form():
    """The exact integer sum against numpy int64 products (a different implementation), and the two float32 products
    in the stated order: (f * sx) * sw differs from f * (sx * sw) on some elements, so the order is pinned."""
    rng = np.random.default_rng(4)
    t, n, k = 13, 37, 640
    xq = rng.integers(-127, 128, (t, k)).astype(np.int8)
    wq = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sx = rng.uniform(1e-3, 1e-1, t).astype(np.float32)
    sw = rng.uniform(1e-3, 1e-1, n).astype(np.float32)
    y = orc.gemm_s8(xq, sx, wq, sw)
    f = (xq.astype(np.int64) @ wq.T.astype(np.int64)).astype(np.float32)
    assert same_bits(orc.gemm_s8(xq, np.ones(t, np.float32), wq, np.ones(n, np.float32)), f)
    left = (f * sx[:, None]).astype(np.float32) * sw[None, :]
    other = f * (sx[:, None] * sw[None, :]).astype(np.float32)
    assert same_bits(y, left.astype(np.float32)) and (other != left).any()


def test_r1_and_r2_differ_on_fp16_weights():
    # the two rules disagree on real data (rounding of w / s against w * (1 / s)): the packer must keep them apart
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((512, 2560)) * 0.02).astype(np.float16).astype(np.float32)
    q1, s1 = orc.quantize_group_r1(w)
    q2, s2 = orc.quantize_block_r2(w)
    assert same_bits(s1, s2)  # same scales where no group is zero
    diff = int((q1 != q2).sum())
    assert 0 < diff < 1000 and np.abs(q1.astype(int) - q2.astype(int)).max() == 1


def test_w8g_chain_against_float64():
    rng = np.random.default_rng(3)
    t, n, k = 9, 64, 512
    x = rng.standard_normal((t, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    q, s = orc.quantize_group_r1(w)
    y = orc.gemm_w8g(x, q, s)
    wd = q.astype(np.float64) * np.repeat(s, 128, axis=1)
    ref = x.astype(np.float64) @ wd.T
    bound = np.abs(x.astype(np.float64)) @ np.abs(wd).T
    assert np.max(np.abs(y - ref) / bound) < 2e-6
    # the group identity sum_g s_g * (sum_k x q) (proofs/GpuTrack/GpuTrack/GroupQuant.lean:38-50)
    grp = sum(s[None, :, g] * (x[:, g * 128:(g + 1) * 128].astype(np.float64) @ q[:, g * 128:(g + 1) * 128].T.astype(np.float64))
              for g in range(k // 128))
    assert max_rel_over_rms(y, grp) < 1e-5
    # Add is one float32 addition onto y
    base = rng.standard_normal((t, n)).astype(np.float32)
    assert same_bits(orc.gemm_w8g(x, q, s, epilogue=orc.ADD, y=base), (base + y).astype(np.float32))
    # SwiGLU on the 64-row interleave: feature 64b + r pairs packed rows 128b + r (gate) and 128b + 64 + r (up)
    gate = (rng.standard_normal((128, k)) / np.sqrt(k)).astype(np.float32)
    up = (rng.standard_normal((128, k)) / np.sqrt(k)).astype(np.float32)
    qW, sW = orc.quantize_group_r1(orc.interleave_gate_up(gate, up))
    ys = orc.gemm_w8g(x, qW, sW, epilogue=orc.SWIGLU)
    plain = orc.gemm_w8g(x, qW, sW)
    for c in (0, 5, 63, 64, 100, 127):
        b_, r_ = divmod(c, 64)
        gv, uv = plain[:, 128 * b_ + r_], plain[:, 128 * b_ + 64 + r_]
        ref_c = np.array([orc.lib().orc_swiglu_libm(float(a_), float(u_)) for a_, u_ in zip(gv, uv)], np.float32)
        assert same_bits(ys[:, c], ref_c)
    # the interleave puts gate row c and up row c together
    qg, sg = orc.quantize_group_r1(gate)
    yg = orc.gemm_w8g(x, qg, sg)
    assert same_bits(plain[:, 128 + 3], yg[:, 64 + 3])


def test_swiglu_forms_against_float64():
    g = np.linspace(-30, 30, 2001).astype(np.float32)
    u = np.linspace(2, -3, 2001).astype(np.float32)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    cep = orc.silu_cephes(g) * u
    libm = np.array([orc.lib().orc_swiglu_libm(float(a), float(b)) for a, b in zip(g, u)], np.float32)
    scale = np.abs(ref) + 1e-3
    assert np.max(np.abs(cep - ref) / scale) < 1e-5
    assert np.max(np.abs(libm - ref) / scale) < 1e-5
    e = orc.exp_cephes(np.linspace(-80, 80, 1001).astype(np.float32)).astype(np.float64)
    ex = np.exp(np.linspace(-80, 80, 1001).astype(np.float32).astype(np.float64))
    assert np.max(np.abs(e - ex) / ex) < 3e-7


def test_gate_up_interleave_order():
    order = orc.gate_up_order(128)
    assert list(order[:64]) == list(range(64)) and list(order[64:128]) == list(range(128, 192))
    assert list(order[128:192]) == list(range(64, 128)) and list(order[192:]) == list(range(192, 256))


@pytest.mark.skipif(not orc.ref_available(), reason="oracle/_ref not built")
def test_oracle_against_live_reference_random_shapes():
    rng = np.random.default_rng(11)
    for t, n, k in [(3, 40, 300), (17, 64, 128), (12, 96, 1000)]:
        x = (rng.standard_normal((t, k)) * 2).astype(np.float32)
        w = (rng.standard_normal((n, k)) * 0.1).astype(np.float32)
        xq, xs = orc.quantize_block_r2(x)
        wq, ws = orc.quantize_block_r2(w)
        assert same_bits(orc.gemm_q8(xq, xs, wq, ws), orc.ref_gemm_i8(x, w))


def test_q8y_matches_reference_avx2_path(golden):
    """kernel_i8_y (runner/src/cpu/gemm_kernels_avx2.cpp): one scale per activation row and per weight feature, both
    from the R2 rule over the whole K; y = ((float)S * ws[n]) * xs[t] then the Store/Add/SwiGLU epilogue."""
    g = golden["ref_i8y"]
    for i in range(int(g["count"])):
        x, w = g[f"c{i}_x"], g[f"c{i}_w"].astype(np.float32)
        k = x.shape[1]
        wq, ws = orc.quantize_block_r2(w, block=k)
        assert same_bits(wq, g[f"c{i}_wq"]) and same_bits(ws.reshape(-1), g[f"c{i}_ws"].reshape(-1))
        xq, xs = orc.quantize_block_r2(x, block=k)
        assert same_bits(orc.gemm_q8y(xq, xs, wq, ws), g[f"c{i}_y"])
        assert same_bits(orc.gemm_q8y(xq, xs, wq, ws, epilogue=orc.ADD, y=g[f"c{i}_base"]), g[f"c{i}_y_acc"])
        if f"c{i}_gate" in g:
            W = orc.interleave_gate_up(g[f"c{i}_gate"].astype(np.float32), g[f"c{i}_up"].astype(np.float32))
            Wq, Ws = orc.quantize_block_r2(W, block=k)
            assert same_bits(orc.gemm_q8y(xq, xs, Wq, Ws, epilogue=orc.SWIGLU), g[f"c{i}_y_swiglu"])
