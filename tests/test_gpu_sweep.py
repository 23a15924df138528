"""A seeded sweep of shapes through the default routing (MI355X only): every path the plan can pick (small-M
streaming, the large-M small-grid plan with and without a K split, the tail-half launches, the 256 x 256 tiles) for
gemm_w8g Store and SwiGLU and gemm_q8 with both activation-scale modes, each against float64 of the dequantized
operands within the bar (max relative error over the elements >= rms < 2e-3, runner/cuda/README.md:113-117)."""
import random
import sys

import pytest

from helpers import max_rel_over_rms

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TS = [1, 2, 5, 15, 16, 17, 31, 32, 33, 48, 63, 64, 65, 100, 129, 200, 300, 511, 700, 1000, 2100]
NS = [16, 48, 128, 384, 1024, 2560, 4096, 12288, 19456]
KS = [128, 256, 1280, 2560, 9728]


def _cases(count, seed):
    rng = random.Random(seed)
    cases = [(t, n, k) for t in TS for n in NS for k in KS]
    rng.shuffle(cases)
    return cases[:count]


@pytest.fixture(scope="module")
def sm():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import sepal_mlp
    sepal_mlp.library()
    return sepal_mlp


@pytest.mark.parametrize("t,n,k", _cases(60, 7))
def test_default_routing_sweep(sm, t, n, k):
    print("[case] sweep", t, n, k, flush=True)
    sys.stdout.flush()
    g = torch.Generator(device="cuda").manual_seed(t * 131 + n * 7 + k)
    w = (torch.randn(n, k, generator=g, device="cuda") * 0.02).half()
    x = torch.randn(t, k, generator=g, device="cuda")
    q, s = sm.quantize_group_s8(w)
    deq = (q.double().view(n, k // 128, 128) * s.double()[:, :, None]).view(n, k)
    xb = x.bfloat16()
    ref = xb.double() @ deq.T
    assert max_rel_over_rms(sm.gemm_w8g(xb, q, s).cpu().numpy(), ref.cpu().numpy()) < 2e-3
    if n % 128 == 0:
        z = ref.view(t, n // 128, 2, 64)
        gate, up = z[:, :, 0, :].reshape(t, n // 2), z[:, :, 1, :].reshape(t, n // 2)
        rs = gate / (1 + torch.exp(-gate)) * up
        ys = sm.gemm_w8g(xb, q, s, epilogue=sm.SWIGLU)
        assert max_rel_over_rms(ys.cpu().numpy(), rs.cpu().numpy()) < 2e-3
    qq, qs = sm.quantize_group_s8(w, rule=sm.RULE_RECIPROCAL)
    deq8 = (qq.double().view(n, k // 128, 128) * qs.double()[:, :, None]).view(n, k)
    for blk in (k, 128):
        xq, xs = sm.quantize_rows_s8(x, block=blk)
        xd = (xq.double().view(t, k // blk, blk) * xs.double()[:, :, None]).view(t, k)
        y8 = sm.gemm_q8(xq, xs, qq, qs, act_block=blk)
        assert max_rel_over_rms(y8.cpu().numpy(), (xd @ deq8.T).cpu().numpy()) < 2e-3, blk
