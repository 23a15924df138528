"""Writes the golden fixtures of the int8 path from the reference's own compiled CPU code (oracle/_ref).

Run in the build container, where /root/reference exists: `make -C oracle && python tests/golden/make_golden.py`.
The fixtures (inputs and the reference's outputs, .npz without pickles) are committed; the tests and the GPU box only
read them. What is dumped:
  ref_suite.npz   the reference test suite's own shapes and inputs (runner/tests/test_cpu_gemm.cpp:84-85, LCG Rng
                  :26-33, x = Rng(5) * 3, w = Rng(6) * 0.5 as in i8_matches_integer_emulation :159-208): pack_weight
                  (q, scale, corr), pack_acts (q, scale), gemm_packed Store and accumulate.
  ref_mlp.npz     MLP-shaped cases with K a multiple of 128 (what the GPU kernels take): gemm_packed Store, Add and the
                  SwiGLU pair (pack_weight_swiglu), weights ~N(0, 0.02), activations ~N(0, 1) with 1% of channels x20.
  ref_rmsnorm.npz rmsnorm_rows with an identity weight and eps 1e-6.
  ref_i8y.npz     the reference's AVX2 int8 path (Variant::I8_Y, kernel_i8_y: one activation scale per row, one
                  weight scale per feature), forced by packing for Isa::Avx2: its weight packing (q, one scale per
                  feature) and gemm_packed Store, Add and SwiGLU, at the suite's odd shapes and at K multiples of 16 and 128;
                  the weights are binary16 values (stored as binary16).
`python tests/golden/make_golden.py i8y` writes ref_i8y.npz only.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import orc  # noqa: E402


def lcg_uniform(seed: int, count: int) -> np.ndarray:
    """The reference test Rng: s = s * 6364136223846793005 + 1442695040888963407; (int32)(s >> 33) / 2^30 - 1."""
    out = np.empty(count, np.float32)
    s = seed
    M = (1 << 64) - 1
    for i in range(count):
        s = (s * 6364136223846793005 + 1442695040888963407) & M
        v = (s >> 33) & 0xFFFFFFFF
        if v >= 1 << 31:
            v -= 1 << 32
        out[i] = np.float32(np.float32(v) / np.float32(1073741824.0) - np.float32(1.0))
    return out


def write_i8y() -> None:
    rng = np.random.default_rng(20261202)
    out = {}
    # weights are binary16 values (stored as such, handed to the reference widened to float32)
    cases = [(13, 37, 70), (29, 100, 129), (37, 128, 256), (130, 128, 512), (16, 128, 1280), (3, 128, 2560),
             (21, 100, 208), (9, 128, 48)]
    half = lambda a: (a * 0.02).astype(np.float16)  # noqa: E731
    for i, (t, n, k) in enumerate(cases):
        x = rng.standard_normal((t, k)).astype(np.float32)
        hot = rng.choice(k, size=max(1, k // 100), replace=False)
        x[:, hot] *= np.float32(20.0)
        x = orc.bf16_round(x)
        w = half(rng.standard_normal((n, k)))
        wf = w.astype(np.float32)
        base = rng.standard_normal((t, n)).astype(np.float32)
        q, s = orc.ref_pack_weight_i8y(wf)
        entry = {"x": x, "w": w, "wq": q, "ws": s, "base": base, "y": orc.ref_gemm_i8y(x, wf),
                 "y_acc": orc.ref_gemm_i8y(x, wf, y=base)}
        if n % 128 == 0:
            gate = half(rng.standard_normal((n // 2, k)))
            up = half(rng.standard_normal((n // 2, k)))
            entry.update({"gate": gate, "up": up,
                          "y_swiglu": orc.ref_gemm_i8y_swiglu(x, gate.astype(np.float32), up.astype(np.float32))})
        out.update({f"c{i}_{name}": v for name, v in entry.items()})
    out["count"] = np.array(len(cases))
    np.savez_compressed(os.path.join(HERE, "ref_i8y.npz"), **out)


def main() -> None:
    if len(sys.argv) > 1 and sys.argv[1] == "i8y":
        write_i8y()
        print("wrote ref_i8y.npz")
        return
    if not orc.ref().ref_i8_variant_is_z():
        raise SystemExit("this CPU does not run the reference's I8_Z kernel (AVX-512 VNNI)")
    # ---- the reference suite's shapes and inputs ----
    shapes = [(1, 1, 1), (5, 7, 3), (13, 37, 70), (29, 100, 129), (96, 64, 256), (50, 33, 1024)]
    suite = {}
    for i, (t, n, k) in enumerate(shapes):
        x = (lcg_uniform(5, t * k) * np.float32(3.0)).reshape(t, k)
        w = (lcg_uniform(6, n * k) * np.float32(0.5)).reshape(n, k)
        q, s, corr = orc.ref_pack_weight_i8(w)
        xq, xs = orc.ref_pack_acts_i8(x)
        y = orc.ref_gemm_i8(x, w)
        base = np.arange(t * n, dtype=np.float32).reshape(t, n) * np.float32(0.01)
        ya = orc.ref_gemm_i8(x, w, y=base)
        for name, v in dict(x=x, w=w, wq=q, ws=s, corr=corr, xq=xq, xs=xs, y=y, y_base=base, y_acc=ya).items():
            suite[f"c{i}_{name}"] = v
    suite["count"] = np.array(len(shapes))
    np.savez_compressed(os.path.join(HERE, "ref_suite.npz"), **suite)

    # ---- MLP-shaped cases ----
    rng = np.random.default_rng(20261201)
    mlp = {}
    cases = [(37, 256, 256), (64, 128, 512), (130, 128, 384), (16, 128, 1280)]
    for i, (t, n, k) in enumerate(cases):
        x = rng.standard_normal((t, k)).astype(np.float32)
        hot = rng.choice(k, size=max(1, k // 100), replace=False)
        x[:, hot] *= np.float32(20.0)
        x = orc.bf16_round(x)
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        gate = (rng.standard_normal((n // 2, k)) * 0.02).astype(np.float32)
        up = (rng.standard_normal((n // 2, k)) * 0.02).astype(np.float32)
        base = rng.standard_normal((t, n)).astype(np.float32)
        mlp.update({f"c{i}_x": x, f"c{i}_w": w, f"c{i}_gate": gate, f"c{i}_up": up, f"c{i}_base": base,
                    f"c{i}_y": orc.ref_gemm_i8(x, w), f"c{i}_y_acc": orc.ref_gemm_i8(x, w, y=base),
                    f"c{i}_y_swiglu": orc.ref_gemm_i8_swiglu(x, gate, up)})
    mlp["count"] = np.array(len(cases))
    np.savez_compressed(os.path.join(HERE, "ref_mlp.npz"), **mlp)

    # ---- RMSNorm ----
    x = (rng.standard_normal((6, 2560)) * 3.0).astype(np.float32)
    x2 = (rng.standard_normal((2, 9728)) * 0.5).astype(np.float32)
    x3 = (rng.standard_normal((5, 136))).astype(np.float32)  # a tail of 8-chunks after the 32-chunks
    np.savez_compressed(os.path.join(HERE, "ref_rmsnorm.npz"), x0=x, y0=orc.ref_rmsnorm(x), x1=x2,
                        y1=orc.ref_rmsnorm(x2), x2=x3, y2=orc.ref_rmsnorm(x3))
    write_i8y()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
