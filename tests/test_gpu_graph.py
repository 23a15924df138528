"""The entry points under HIP graph capture (MI355X only): a stream whose workspace is sized by warm-up calls records no
allocation and no memset, so a captured sequence replays. Each graph is replayed several times with eager work of
the library on another stream between the replays, and every replay's outputs must equal the eager results bit for
bit (split-K counters return to zero at the end of every call, so a replay starts from the same state)."""
import sys

import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def sm():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import sepal_mlp
    sepal_mlp.library()
    return sepal_mlp


_SIDE = []


def _side():
    """One side stream for every test of the module (the library keeps a workspace per stream)."""
    if not _SIDE:
        _SIDE.append(torch.cuda.Stream())
    return _SIDE[0]


# T = 1 and 16: the pass kernels; 48: the large-M plan with a K split; 896: split-K down, planned gate/up
@pytest.mark.parametrize("t", [1, 16, 48, 896])
def test_captured_mlp_block_replays(sm, t):
    say("graph replay", t)
    H, I = 2560, 9728
    g = torch.Generator(device="cuda").manual_seed(77 + t)
    gate = (torch.randn(I, H, generator=g, device="cuda") * 0.02).half()
    up = (torch.randn(I, H, generator=g, device="cuda") * 0.02).half()
    down = (torch.randn(H, I, generator=g, device="cuda") * 0.02).half()
    wgu, sgu = sm.quantize_gate_up_s8(gate, up)
    wd, sd = sm.quantize_group_s8(down)
    qgu, qsgu = sm.quantize_gate_up_s8(gate, up, rule=sm.RULE_RECIPROCAL)
    qd, qsd = sm.quantize_group_s8(down, rule=sm.RULE_RECIPROCAL)
    x = torch.randn(t, H, generator=g, device="cuda")
    xb = x.bfloat16()
    h = torch.empty(t, I, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(t, H, device="cuda")
    hf = torch.empty(t, I, device="cuda")
    z = torch.empty(t, H, device="cuda")
    xq = torch.empty(t, H, dtype=torch.int8, device="cuda")
    xs = torch.empty(t, 1, device="cuda")

    def block(st):
        sm.gemm_w8g(xb, wgu, sgu, y=h, epilogue=sm.SWIGLU, stream=st)
        sm.gemm_w8g(h, wd, sd, y=y, stream=st)
        q, s_ = sm.quantize_rows_s8(x, block=H, stream=st)
        xq.copy_(q)
        xs.copy_(s_)
        sm.gemm_q8(xq, xs, qgu, qsgu, y=hf, epilogue=sm.SWIGLU, act_block=H, stream=st)
        hq, hs = sm.quantize_rows_s8(hf, block=I, stream=st)
        sm.gemm_q8(hq, hs, qd, qsd, y=z, act_block=I, stream=st)

    side = _side()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            block(side)
    torch.cuda.synchronize()
    y_ref, z_ref, h_ref = y.clone(), z.clone(), h.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        block(side)
    for i in range(3):
        y.zero_()
        z.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(h, h_ref) and torch.equal(y, y_ref) and torch.equal(z, z_ref), i
        # eager work of the library between the replays (its own stream and workspace)
        sm.gemm_w8g(xb, wgu, sgu, epilogue=sm.SWIGLU)
        torch.cuda.synchronize()
