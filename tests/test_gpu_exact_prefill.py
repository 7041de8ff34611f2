"""EXACT above 1024 picks: gfl_moe_forward with prefill-sized batches (the decode kernels driven by the grouped plan)
against the oracle's EXACT layer forward, bit for bit.

The reference's EXACT moe_forward (kernels/cpu_avx2/ft_core.h:1338-1407) has no batch limit; its jobs (8 tokens of one
expert each, first-appearance order) fix every token's combine order over the whole batch, so each case compares the
full call (or, at the largest sizes, chosen rows evaluated with the whole batch's jobs: oracle.moe_forward_rows).
"""
import numpy as np
import pytest


def _layer(gpu, li, E, H, I, Ks=(3, 3, 3)):
    import synth
    L = synth.SynthLayer(li, E, H, I, Ks)
    L.register(gpu, li)
    return L


def _mats(L, ids):
    from oracle import Mat
    out = {}
    for e in ids:
        ms = []
        for p in range(3):
            tr, suh, svh = L.matrix(e, p)
            k, n = (L.H, L.I) if p < 2 else (L.I, L.H)
            ms.append(Mat(tr, suh, svh, k, n, L.Ks[p]))
        out[e] = tuple(ms)
    return out


def _forward(gpu, li, x16, sel, w):
    import torch
    xd = torch.from_numpy(x16.view(np.int16)).view(torch.float16).cuda()
    seld = torch.from_numpy(np.ascontiguousarray(sel, dtype=np.int64)).cuda()
    wd = torch.from_numpy(np.ascontiguousarray(w)).cuda()
    out = torch.full(x16.shape, float("nan"), dtype=torch.float32, device="cuda")
    gpu.moe_forward(li, xd.contiguous(), seld, wd, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _route(kind, M, topk, E, rng):
    if kind == "uniform":
        return np.stack([rng.permutation(E)[:topk] for _ in range(M)]).astype(np.int64)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    sel = rng.choice(E, size=(M, topk), p=p / p.sum()).astype(np.int64)   # repeats within a token
    if kind == "bad":
        m = rng.random(sel.shape)
        sel[m < 0.1] = -1
        sel[(m >= 0.1) & (m < 0.12)] = E + 3
        sel[5] = -1                                                       # a token without any valid pick
    return sel


@pytest.mark.gpu
@pytest.mark.parametrize("M,topk,E,kind,Ks", [
    (129, 8, 16, "uniform", (3, 3, 3)),     # 1,032 picks: just above the decode plan's limit
    (700, 6, 40, "bad", (3, 3, 3)),         # skipped, out-of-range and repeated ids, an empty token
    (300, 8, 12, "zipf", (4, 4, 3)),        # config-2 layer A bitrates
    (300, 8, 12, "zipf", (3, 3, 5)),        # config-2 layer B bitrates
    (260, 4, 9, "uniform", (2, 5, 4)),      # gate and up at different K (two gate|up launches)
])
def test_exact_above_1024_picks_bitexact(gpu, oracle, M, topk, E, kind, Ks):
    H, I, li = 512, 256, 60
    L = _layer(gpu, li, E, H, I, Ks)
    rng = np.random.default_rng(M * 7 + topk)
    x16 = (rng.standard_normal((M, H)) * 0.4).astype(np.float16)
    sel = _route(kind, M, topk, E, rng)
    w = rng.random(sel.shape).astype(np.float32)
    print(f"EXACT large: M={M} topk={topk} E={E} {kind} K={Ks}", flush=True)
    got = _forward(gpu, li, x16, sel, w)
    m = _mats(L, range(E))
    osel = np.where((sel >= 0) & (sel < E), sel, -1)
    want = oracle.moe_forward([m[e] for e in range(E)], x16.astype(np.float32), osel, w, mode=1)
    nbad = int(np.count_nonzero(got != want))
    print(f"  mismatched {nbad}/{want.size}")
    assert nbad == 0
    if kind == "bad":
        assert np.all(got[5] == 0.0)


@pytest.mark.gpu
def test_exact_at_the_pick_maximum_rows_bitexact(gpu, oracle):
    """65,536 picks (M=4096, top-16 of 64 experts, Zipf with repeats): eight rows spread over the batch against the
    oracle with the whole batch's jobs."""
    H, I, E, M, topk, li = 512, 256, 64, 4096, 16, 61
    L = _layer(gpu, li, E, H, I)
    rng = np.random.default_rng(65536)
    x16 = (rng.standard_normal((M, H)) * 0.4).astype(np.float16)
    sel = _route("zipf", M, topk, E, rng)
    w = rng.random(sel.shape).astype(np.float32)
    got = _forward(gpu, li, x16, sel, w)
    assert np.isfinite(got).all()
    rows = [0, 1, 999, 2048, 3000, 4000, 4094, 4095]
    need = sorted(set(int(e) for r in rows for e in sel[r]))
    m = _mats(L, need)
    ex = [m.get(e, m[need[0]]) for e in range(E)]   # experts no wanted row picks are never read
    want = oracle.moe_forward_rows(ex, x16.astype(np.float32), sel, w, rows, mode=1)
    nbad = int(np.count_nonzero(got[rows] != want))
    print(f"EXACT 65536 picks, rows {rows}: mismatched {nbad}/{want.size}")
    assert nbad == 0


@pytest.mark.gpu
def test_exact_large_graph_replay(gpu):
    """Workspace reserved up front (gfl_grouped_reserve), then an M=300 top-8 EXACT call captured in a HIP graph and
    replayed three times with eager calls between: a decode-sized one, one above 1,024 picks within the reserve, and
    one above the reserved 4,096 picks, which grows the prefill workspace (the captured graph keeps the retired
    buffer's addresses). Every replay equals the eager result."""
    import torch
    H, I, E, li = 512, 256, 16, 62
    _layer(gpu, li, E, H, I)
    gpu.grouped_reserve(4096)
    rng = np.random.default_rng(62)
    M = 300
    x = torch.from_numpy((rng.standard_normal((M, H)) * 0.4).astype(np.float16)).cuda()
    sel = torch.from_numpy(_route("zipf", M, 8, E, rng)).cuda()
    w = torch.from_numpy(rng.random((M, 8)).astype(np.float32)).cuda()
    ref = torch.empty((M, H), dtype=torch.float32, device="cuda")
    gpu.moe_forward(li, x, sel, w, ref)
    torch.cuda.synchronize()
    out = torch.zeros_like(ref)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            gpu.moe_forward(li, x, sel, w, out)
    torch.cuda.synchronize()
    other = torch.empty_like(ref)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        gpu.moe_forward(li, x[:50], sel[:50], w[:50], other[:50])   # an eager call in between (other sizes)
        torch.cuda.synchronize()
    # eager calls of the prefill path between replays: 1,600 picks inside the reserve, then 4,800 beyond it
    xb = torch.from_numpy((rng.standard_normal((600, H)) * 0.4).astype(np.float16)).cuda()
    sb = torch.from_numpy(_route("zipf", 600, 8, E, rng)).cuda()
    wb = torch.from_numpy(rng.random((600, 8)).astype(np.float32)).cuda()
    big = torch.empty((600, H), dtype=torch.float32, device="cuda")
    for m in (200, 600):
        gpu.moe_forward(li, xb[:m], sb[:m], wb[:m], big[:m])
        torch.cuda.synchronize()
        assert torch.all(torch.isfinite(big[:m]))
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay after an eager call of {m * 8} picks"
