"""Shared checks of the parity tests."""
from __future__ import annotations

import numpy as np


def max_rel_over_rms(got, ref) -> float:
    """The reference's parity measure (runner/cuda/README.md:113-117): the largest elementwise relative difference over
    the elements at least as large as the rms of the reference."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref * ref))
    big = np.abs(ref) >= rms
    if not big.any():
        return 0.0
    return float(np.max(np.abs(got[big] - ref[big]) / np.abs(ref[big])))


def rel_rms(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.sqrt(np.mean((got - ref) ** 2) / max(np.mean(ref * ref), 1e-300)))


def same_bits(a, b) -> bool:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and a.tobytes() == b.tobytes()


def bf16_inputs(rng, shape, outlier_frac: float = 0.0, scale: float = 1.0):
    """float32 values that are exact bfloat16 (~N(0, scale^2), a fraction of channels x20 before rounding)."""
    from oracle import orc
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    if outlier_frac > 0:
        k = shape[-1]
        hot = rng.choice(k, size=max(1, int(round(k * outlier_frac))), replace=False)
        x[..., hot] *= np.float32(20.0)
    return orc.bf16_round(x)


def per_token_layer_stages(sm, x, layer, rows=None):
    """One q8 layer with one activation scale per token, stage by stage against the oracle: X quantized bit for bit;
    H (binary16, the SwiGLU the fast one: no reference bits to match) within the bar of the oracle's float32 H; H
    quantized per token bit for bit from the GPU's own H; the down multiply on the GPU's own int8 H bit for bit (above
    64 rows; below, at float32 rounding: the small-M kernels add partial chains of the same int32 sums). End
    to end, a binary16 H moves an activation across an int8 rounding boundary once in ~5e4 values where the oracle's
    H rounds the other way, and each such step moves its row by up to ~4e-3 at K = 512, so the end-to-end comparison
    is held to the bar in relative rms (the stages above carry the exactness)."""
    import torch

    from oracle import orc

    def dev(a, dtype):
        return torch.from_numpy(np.ascontiguousarray(a)).cuda().to(dtype)

    def host(t):
        torch.cuda.synchronize()
        return t.cpu().numpy()

    wgu, sgu, wd, sd = layer
    hidden, inter = x.shape[1], wd.shape[1]
    rows = np.arange(x.shape[0]) if rows is None else rows
    xq_g, xs_g = sm.quantize_rows_s8(dev(x, torch.bfloat16), block=hidden)
    xq, xs = orc.quantize_block_r2(x[rows], block=hidden)
    assert same_bits(host(xq_g)[rows], xq) and same_bits(host(xs_g).reshape(-1)[rows], xs.reshape(-1))
    hg = sm.gemm_q8(xq_g, xs_g, wgu, sgu, epilogue=sm.SWIGLU, act_block=hidden, y_dtype=torch.float16)
    h_g = host(hg.float())
    h = orc.gemm_q8(xq, xs, host(wgu), host(sgu), epilogue=orc.SWIGLU, act_block=hidden)
    assert max_rel_over_rms(h_g[rows], h) < 2e-3, max_rel_over_rms(h_g[rows], h)
    hq_g, hs_g = sm.quantize_rows_s8(hg, block=inter)
    hq, hs = orc.quantize_block_r2(h_g[rows], block=inter)
    assert same_bits(host(hq_g)[rows], hq) and same_bits(host(hs_g).reshape(-1)[rows], hs.reshape(-1))
    y_g = host(sm.gemm_q8(hq_g, hs_g, wd, sd, act_block=inter))
    y_o = orc.gemm_q8(hq, hs, host(wd), host(sd), act_block=inter)
    if x.shape[0] > 64:
        assert same_bits(y_g[rows], y_o)  # the large-M kernels chain the groups in the reference's order
    else:
        # (up to 64 rows the small-M kernels add partial chains of the same exact int32 sums: float32 rounding)
        assert max_rel_over_rms(y_g[rows], y_o) < 1e-5, max_rel_over_rms(y_g[rows], y_o)
    return y_g
