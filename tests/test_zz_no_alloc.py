"""gfl_moe_forward_noalloc (the decode forward on the library's static scratch array) against gfl_moe_forward.

Bar: bit-identical outputs on the same inputs, for two calls in a row with the second smaller, in EXACT and MFMA
modes; sizes beyond the array's layout are refused; the calls allocate no device memory.
"""
import numpy as np
import pytest

import _native


def _inputs(rng, M, topk, E, H):
    import torch
    x = torch.from_numpy((rng.standard_normal((M, H)) * 0.35).astype(np.float16)).cuda()
    sel = torch.from_numpy(np.stack([rng.choice(E, topk, replace=False) for _ in range(M)]).astype(np.int64)).cuda()
    w = torch.from_numpy(rng.random((M, topk)).astype(np.float32)).cuda()
    return x, sel, w


def _pair(gpu, li, x, sel, w, mode):
    import torch
    want = torch.empty(x.shape, dtype=torch.float32, device="cuda")
    got = torch.full(x.shape, float("nan"), dtype=torch.float32, device="cuda")
    gpu.moe_forward(li, x, sel, w, want, mode=mode)
    gpu.moe_forward_noalloc(li, x, sel, w, got, mode=mode)
    torch.cuda.synchronize()
    return got.cpu().numpy(), want.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [_native.MODE_EXACT, _native.MODE_MFMA])
def test_noalloc_matches_forward_two_calls(gpu, mode):
    import torch
    import synth
    H, I, E, topk, li = 5120, 1536, 96, 8, 950
    synth.SynthLayer(li, E, H, I, (4, 4, 3)).register(gpu, li)
    rng = np.random.default_rng(4242 + mode)
    # 64 picks (the maximum), then fewer: 24 and 8 (in EXACT mode the relay launches with one and two waves per
    # gate|up column), then 8 again on the context told that it shares the GPU (the per-slot launches)
    cases = [_inputs(rng, M, topk, E, H) for M in (8, 3, 1, 1)]
    _pair(gpu, li, *cases[0], mode)                         # kernels loaded, output tensors cached by torch
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    try:
        for i, (x, sel, w) in enumerate(cases):
            shared = i == len(cases) - 1
            gpu.set_shared(shared)
            print(f"noalloc mode={mode} call {i}: M={x.shape[0]} topk={topk} H={H} I={I} shared={shared}", flush=True)
            got, want = _pair(gpu, li, x, sel, w, mode)
            nbad = int(np.count_nonzero(got != want))
            print(f"  mismatched {nbad}/{want.size}, max-abs {float(np.abs(got - want).max()):.3e}", flush=True)
            assert np.all(np.isfinite(want)) and nbad == 0
    finally:
        gpu.set_shared(False)
    assert torch.cuda.mem_get_info()[0] == free0


@pytest.mark.gpu
def test_noalloc_small_shape_and_limits(gpu):
    import torch
    import synth
    H, I, E, li = 512, 256, 6, 951
    synth.SynthLayer(li, E, H, I, (3, 3, 3)).register(gpu, li)
    rng = np.random.default_rng(99)
    for M, topk in [(9, 4), (1, 4), (16, 4)]:
        x, sel, w = _inputs(rng, M, topk, E, H)
        got, want = _pair(gpu, li, x, sel, w, _native.MODE_EXACT)
        assert np.array_equal(got, want), (M, topk)
    x, sel, w = _inputs(rng, 17, 4, E, H)   # 68 picks: beyond the static layout
    out = torch.empty(x.shape, dtype=torch.float32, device="cuda")
    with pytest.raises(_native.NativeError, match="M\\*topk <= 64"):
        gpu.moe_forward_noalloc(li, x, sel, w, out)


@pytest.mark.gpu
def test_noalloc_graph_replays(gpu):
    """A no-allocation call captured into a HIP graph (torch.cuda.graph) replays to the eager result, with eager
    no-allocation calls of other sizes and a gfl_moe_forward call run between the replays."""
    import torch
    import synth
    H, I, E, li = 512, 256, 6, 952
    synth.SynthLayer(li, E, H, I, (3, 3, 3)).register(gpu, li)
    rng = np.random.default_rng(123)
    x, sel, w = _inputs(rng, 2, 4, E, H)
    want = torch.empty(x.shape, dtype=torch.float32, device="cuda")
    gpu.moe_forward(li, x, sel, w, want)
    out = torch.full(x.shape, float("nan"), dtype=torch.float32, device="cuda")
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        gpu.moe_forward_noalloc(li, x, sel, w, out)       # warm-up on a side stream, as torch's graph recipe does
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gpu.moe_forward_noalloc(li, x, sel, w, out)
    others = [_inputs(rng, M, 4, E, H) for M in (9, 1)]
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep}"
        xo, so, wo = others[rep % 2]
        a = torch.empty(xo.shape, dtype=torch.float32, device="cuda")
        b = torch.empty(xo.shape, dtype=torch.float32, device="cuda")
        gpu.moe_forward_noalloc(li, xo, so, wo, a)          # eager work between the replays
        gpu.moe_forward(li, xo, so, wo, b)
        torch.cuda.synchronize()
        assert torch.equal(a, b)
    del g
