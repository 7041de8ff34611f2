"""The shared expert on a side stream (k_overlap.SharedOverlap, the counterpart of glm53/k_overlap.py) against the CPU
oracle: the overlapped result equals the routed layer plus the shared expert, each computed in the reference's EXACT
mode, added in fp32 (bit-exact); the sequential order gives the same bits; the fork/join captures into a HIP graph
whose replays (with eager work and synchronisations between them) reproduce the eager results."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

H, I, E = 512, 256, 6


def _experts(L):
    from oracle import Mat
    out = []
    for e in range(L.E):
        mats = []
        for p in range(3):
            tr, suh, svh = L.matrix(e, p)
            k, n = (L.H, L.I) if p < 2 else (L.I, L.H)
            mats.append(Mat(tr, suh, svh, k, n, L.Ks[p]))
        out.append(tuple(mats))
    return out


@pytest.fixture(scope="module")
def setup(gpu):
    import k_overlap
    import synth
    li = 61
    routed = synth.SynthLayer(li, E, H, I, (3, 3, 3))
    routed.register(gpu, li)
    shared = synth.SynthLayer(62, 1, H, I, (4, 4, 3))
    so = k_overlap.SharedOverlap(0)
    so.register(li, H, I, shared.Ks, shared.ptr_table, keep=shared)
    return dict(li=li, routed=routed, shared=shared, so=so)


def _inputs(rng, M):
    import torch
    x16 = (rng.standard_normal((M, H)) * 0.5).astype(np.float16)
    sel = np.stack([rng.permutation(E)[:3] for _ in range(M)]).astype(np.int64)
    w = rng.random(sel.shape).astype(np.float32)
    t = (torch.from_numpy(x16.view(np.int16)).view(torch.float16).cuda(), torch.from_numpy(sel).cuda(),
         torch.from_numpy(w).cuda())
    return x16, sel, w, t


@pytest.mark.parametrize("M", [1, 17, 33])
def test_overlap_equals_routed_plus_shared(gpu, oracle, setup, M):
    """The three orders SharedOverlap takes (96 routed gate|up tile columns per token here): M = 1 runs in the stock
    order (at most 1,536 columns), M = 17 (1,632) overlaps the shared expert on its own launches, M = 33 (3,168) on
    its narrower ones."""
    import torch
    rng = np.random.default_rng(70 + M)
    x16, sel, w, (xd, seld, wd) = _inputs(rng, M)
    out = torch.empty((M, H), dtype=torch.float32, device="cuda")
    before = setup["so"].summary()
    setup["so"].forward(gpu, setup["li"], xd, seld, wd, out)
    torch.cuda.synchronize()
    after = setup["so"].summary()
    took = "sequential" if M == 1 else "overlapped"
    assert after[took] == before[took] + 1
    got = out.cpu().numpy()
    routed = oracle.moe_forward(_experts(setup["routed"]), x16.astype(np.float32), sel, w, mode=1)
    shared = oracle.expert_forward(_experts(setup["shared"])[0], x16.astype(np.float32), mode=1)
    want = (routed.astype(np.float32) + shared.astype(np.float32)).astype(np.float32)
    assert np.array_equal(got, want)
    seq = torch.empty_like(out)
    setup["so"].forward(gpu, setup["li"], xd, seld, wd, seq, overlap=False)
    torch.cuda.synchronize()
    assert np.array_equal(seq.cpu().numpy(), got)
    # the routed context's own shared flag survives the overlapped call, whichever it was
    for flag in (True, False):
        gpu.set_shared(flag)
        setup["so"].forward(gpu, setup["li"], xd, seld, wd, out)
        assert gpu.shared is flag


def test_overlap_graph_replays(gpu, setup):
    """M = 17: the overlapped order (fork, side stream, join) inside a captured graph."""
    import torch
    rng = np.random.default_rng(80)
    M = 17
    ins = [_inputs(rng, M)[3] for _ in range(3)]
    outs = [torch.empty((M, H), dtype=torch.float32, device="cuda") for _ in range(3)]
    for (xd, seld, wd), o in zip(ins, outs):
        setup["so"].forward(gpu, setup["li"], xd, seld, wd, o)
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        setup["so"].forward(gpu, setup["li"], *ins[0], outs[0])
    torch.cuda.current_stream().wait_stream(st)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for (xd, seld, wd), o in zip(ins, outs):
            setup["so"].forward(gpu, setup["li"], xd, seld, wd, o)
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep}"
        setup["so"].forward(gpu, setup["li"], *ins[1], outs[1])      # eager work between replays
        torch.cuda.synchronize()
    del g
