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


# ---- the shared expert in the routed call's own launches (gfl_moe_forward_shared) ----

def _ctx_env(**env):
    """A context created under the given environment (GFL_RELAY is read once, at creation)."""
    import os
    import _native
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return _native.Context(0)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def _want(oracle, routed, shared, x16, sel, w):
    r = oracle.moe_forward(_experts(routed), x16.astype(np.float32), sel, w, mode=1)
    s = oracle.expert_forward(_experts(shared)[0], x16.astype(np.float32), mode=1)
    return (r.astype(np.float32) + s.astype(np.float32)).astype(np.float32)


@pytest.mark.parametrize("relay", [None, "1,1", "2,1", "4,4", "2,2"])
def test_fused_shared_bitexact(gpu, oracle, relay):
    """routed + shared in one call's launches equals the routed layer plus the shared expert (fp32 add after the routed
    sum), bit for bit: M = 1, 2, 5, 8 at top-3 of 6 experts, with a skipped pick, a token picking one expert twice and
    a token whose picks are all skipped (its row is the shared expert alone); relay widths as chosen or forced."""
    import torch
    import synth
    ctx = gpu if relay is None else _ctx_env(GFL_RELAY=relay)
    li = 63
    routed = synth.SynthLayer(li, E, H, I, (3, 4, 3))
    routed.register(ctx, li)
    shared = synth.SynthLayer(64, 1, H, I, (3, 4, 3))
    ctx.register_shared(li, shared.Ks, shared.ptr_table, keep=shared)
    for M in (1, 2, 5, 8):
        rng = np.random.default_rng(90 + M)
        x16, sel, w, _ = _inputs(rng, M)
        if M >= 2:
            sel[0, 2] = -1
            sel[1, :] = -1
        if M >= 5:
            sel[3, 1] = sel[3, 0]
        xd = torch.from_numpy(x16.view(np.int16)).view(torch.float16).cuda()
        out = torch.full((M, H), float("nan"), dtype=torch.float32, device="cuda")
        assert ctx.moe_forward_shared(li, xd, torch.from_numpy(sel).cuda(), torch.from_numpy(w).cuda(), out)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), _want(oracle, routed, shared, x16, sel, w)), f"M={M}"


def test_fused_shared_act_limit(gpu, oracle):
    """The SwiGLU clamp reaches the shared expert too: the fused call with act_limit equals the routed layer and the
    shared expert each computed with that clamp, added after the routed sum."""
    import torch
    import synth
    li = 72
    routed = synth.SynthLayer(li, E, H, I, (3, 3, 3))
    routed.register(gpu, li)
    shared = synth.SynthLayer(73, 1, H, I, (3, 3, 3))
    gpu.register_shared(li, shared.Ks, shared.ptr_table, keep=shared)
    lim = 0.05
    rng = np.random.default_rng(97)
    x16, sel, w, (xd, seld, wd) = _inputs(rng, 3)
    out = torch.full((3, H), float("nan"), dtype=torch.float32, device="cuda")
    assert gpu.moe_forward_shared(li, xd, seld, wd, out, act_limit=lim)
    torch.cuda.synchronize()
    r = oracle.moe_forward(_experts(routed), x16.astype(np.float32), sel, w, mode=1, act_limit=lim)
    sh = oracle.expert_forward(_experts(shared)[0], x16.astype(np.float32), mode=1, act_limit=lim)
    assert np.array_equal(out.cpu().numpy(), (r.astype(np.float32) + sh.astype(np.float32)).astype(np.float32))


def test_fused_shared_declines(gpu):
    """gfl_moe_forward_shared launches nothing and says so (False) for calls it cannot fuse: the shared expert's bit
    widths differ from the layer's, mode MFMA, more than 64 routed picks; a layer without a shared expert is an error."""
    import torch
    import synth
    import _native
    li = 65
    routed = synth.SynthLayer(li, E, H, I, (3, 3, 3))
    routed.register(gpu, li)
    rng = np.random.default_rng(99)
    x16, sel, w, (xd, seld, wd) = _inputs(rng, 2)
    out = torch.full((2, H), float("nan"), dtype=torch.float32, device="cuda")
    with pytest.raises(_native.NativeError):
        gpu.moe_forward_shared(li, xd, seld, wd, out)
    other = synth.SynthLayer(66, 1, H, I, (4, 4, 3))
    gpu.register_shared(li, other.Ks, other.ptr_table, keep=other)
    assert not gpu.moe_forward_shared(li, xd, seld, wd, out)
    same = synth.SynthLayer(67, 1, H, I, (3, 3, 3))
    gpu.register_shared(li, same.Ks, same.ptr_table, keep=same)
    assert not gpu.moe_forward_shared(li, xd, seld, wd, out, mode=_native.MODE_MFMA)
    _, _, _, (xb, selb, wb) = _inputs(rng, 22)   # 66 routed picks
    outb = torch.full((22, H), float("nan"), dtype=torch.float32, device="cuda")
    assert not gpu.moe_forward_shared(li, xb, selb, wb, outb)
    torch.cuda.synchronize()
    assert torch.isnan(out).all() and torch.isnan(outb).all()
    assert gpu.moe_forward_shared(li, xd, seld, wd, out)


def test_fused_shared_full_shape_bitexact(gpu, oracle):
    """The config-1 shape (H=5120, I=1536, K=3), top-8 of a 10-expert layer plus a shared expert at M = 1 and 3 (9 and
    27 picks through the relay launches)."""
    import torch
    import synth
    Hf, If, Ef = 5120, 1536, 10
    li = 68
    routed = synth.SynthLayer(li, Ef, Hf, If, (3, 3, 3))
    routed.register(gpu, li)
    shared = synth.SynthLayer(69, 1, Hf, If, (3, 3, 3))
    gpu.register_shared(li, shared.Ks, shared.ptr_table, keep=shared)
    for M in (1, 3):
        rng = np.random.default_rng(95 + M)
        x16 = rng.standard_normal((M, Hf)).astype(np.float16)
        (sel, w16), _ = synth.route_uniform(M, Ef, 8, rng)
        out = torch.full((M, Hf), float("nan"), dtype=torch.float32, device="cuda")
        assert gpu.moe_forward_shared(li, torch.from_numpy(x16.view(np.int16)).view(torch.float16).cuda(),
                                      torch.from_numpy(sel).cuda(),
                                      torch.from_numpy(w16.view(np.int16)).view(torch.float16).cuda(), out)
        torch.cuda.synchronize()
        want = _want(oracle, routed, shared, x16, sel, w16.astype(np.float32))
        assert np.array_equal(out.cpu().numpy(), want), f"M={M}"


def test_shared_overlap_fuses(gpu, oracle):
    """SharedOverlap with the routed context holding the shared expert runs both in one call (summary "fused") and
    gives the stock order's bits; the graph of such calls replays to the eager results."""
    import torch
    import k_overlap
    import synth
    li = 70
    routed = synth.SynthLayer(li, E, H, I, (3, 3, 3))
    routed.register(gpu, li)
    shared = synth.SynthLayer(71, 1, H, I, (3, 3, 3))
    so = k_overlap.SharedOverlap(0)
    so.register(li, H, I, shared.Ks, shared.ptr_table, keep=shared, routed=gpu)
    rng = np.random.default_rng(98)
    x16, sel, w, (xd, seld, wd) = _inputs(rng, 4)
    out = torch.empty((4, H), dtype=torch.float32, device="cuda")
    so.forward(gpu, li, xd, seld, wd, out)
    assert so.summary()["fused"] == 1
    seq = torch.empty_like(out)
    so.forward(gpu, li, xd, seld, wd, seq, overlap=False)
    torch.cuda.synchronize()
    assert torch.equal(out, seq)
    assert np.array_equal(out.cpu().numpy(), _want(oracle, routed, shared, x16, sel, w))
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        so.forward(gpu, li, xd, seld, wd, out)
    torch.cuda.current_stream().wait_stream(st)
    with torch.cuda.graph(g):
        so.forward(gpu, li, xd, seld, wd, out)
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, seq), f"replay {rep}"
        so.forward(gpu, li, xd, seld, wd, seq, overlap=False)   # eager work between replays
        torch.cuda.synchronize()
    del g
