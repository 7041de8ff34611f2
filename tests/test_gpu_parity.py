"""HIP path vs the CPU oracle, through the C ABI (libgfl_moe.so).

Bar: dequantized weights bit-exact; expert and layer outputs bit-exact against the reference's EXACT mode (the
oracle restates it bit-for-bit, see test_oracle.py). Every case also reports max-abs/RMS against the north-star
tolerance (max|y - y_ref| <= 2e-3 * RMS(y_ref)), which bit-exactness implies.
"""
import numpy as np
import pytest

TOL = 2e-3   # north-star: max-abs error relative to output RMS


def _layer(gpu, li, E, H, I, Ks=(3, 3, 3)):
    import synth
    L = synth.SynthLayer(li, E, H, I, Ks)
    L.register(gpu, li)
    return L


def _host_experts(oracle, L):
    from oracle import Mat
    ex = []
    for e in range(L.E):
        mats = []
        for p in range(3):
            tr, suh, svh = L.matrix(e, p)
            k, n = (L.H, L.I) if p < 2 else (L.I, L.H)
            mats.append(Mat(tr, suh, svh, k, n, L.Ks[p]))
        ex.append(tuple(mats))
    return ex


def _forward(gpu, li, x16, sel, w, w_half=False):
    import torch
    xd = torch.from_numpy(x16.view(np.int16)).view(torch.float16).cuda()
    seld = torch.from_numpy(np.ascontiguousarray(sel, dtype=np.int64)).cuda()
    wd = torch.from_numpy(np.ascontiguousarray(w)).cuda()
    out = torch.empty(x16.shape, dtype=torch.float32, device="cuda")
    gpu.moe_forward(li, xd.contiguous(), seld, wd, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _report(name, got, want):
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    mx = float(np.abs(got.astype(np.float64) - want).max())
    nbad = int(np.count_nonzero(got != want))
    print(f"{name}: max-abs {mx:.3e} rms {rms:.3e} ratio {mx / max(rms, 1e-30):.3e} mismatched {nbad}/{want.size}")
    return mx, rms, nbad


@pytest.mark.gpu
@pytest.mark.parametrize("K", [3, 4, 5, 2])
def test_dequant_bitexact(gpu, oracle, K):
    import torch
    import synth
    import _native
    for (k, n, s) in [(256, 128, 11), (512, 384, 12), (5120, 1536, 13)]:
        nb = synth.trellis_bytes(k, n, K)
        tr = torch.empty(nb, dtype=torch.uint8, device="cuda")
        _native.synth_trellis(tr, s)
        W = torch.empty((k, n), dtype=torch.int16, device="cuda")
        _native.dequant(tr, k, n, K, W)
        torch.cuda.synchronize()
        got = W.cpu().numpy().view(np.uint16)
        want = oracle.dequant(tr.cpu().numpy(), k, n, K)
        print(f"dequant K={K} {k}x{n}: mismatches {int(np.count_nonzero(got != want))}")
        assert np.array_equal(got, want)


@pytest.mark.gpu
def test_synth_trellis_matches_checker(gpu, oracle):
    import torch
    import _native
    for nb, s in [(96, 1), (1000, 2), (8847, 0x6A11F1A5)]:
        t = torch.empty(nb, dtype=torch.uint8, device="cuda")
        _native.synth_trellis(t, s)
        torch.cuda.synchronize()
        assert np.array_equal(t.cpu().numpy(), oracle.synth_trellis(s, nb))


@pytest.mark.gpu
@pytest.mark.parametrize("ntok", [1, 3, 4, 8, 9])
def test_forward_small_bitexact(gpu, oracle, ntok):
    """Small shape, the reference harness's routing (t + 2k) % E (duplicate picks of one expert per token). Up to 8
    tokens the launches run a workgroup per slot, from 9 a workgroup per expert with passes of two slots."""
    H, I, E = 512, 256, 6
    L = _layer(gpu, 1, E, H, I)
    ex = _host_experts(oracle, L)
    rng = np.random.default_rng(777 + ntok)
    x16 = (rng.standard_normal((ntok, H)) * 0.35).astype(np.float16)
    sel = np.array([[(t + 2 * k) % E for k in range(4)] for t in range(ntok)], np.int64)
    w = np.full(sel.shape, 0.25, np.float32)
    got = _forward(gpu, 1, x16, sel, w)
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1)
    mx, rms, nbad = _report(f"small ntok={ntok}", got, want)
    assert nbad == 0


@pytest.mark.gpu
@pytest.mark.parametrize("nt", [1, 3, 4, 16])
def test_forward_equals_reference_engine_golden(gpu, nt):
    """Layer output against the reference engine's own EXACT moe_forward (tests/golden, written from
    kernels/cpu_avx2/ft_core.h), no oracle in between: H=512 I=256 E=6, harness routing (t + 2k) % 6, weight 0.25;
    16 tokens give every expert two jobs."""
    import os
    from conftest import GOLDEN
    G = np.load(os.path.join(GOLDEN, "ref_vectors.npz"))
    _layer(gpu, 7, 6, 512, 256)
    x, sel = G[f"moe_x_{nt}"], G[f"moe_sel_{nt}"].astype(np.int64)
    w = np.full(sel.shape, 0.25, np.float32)
    got = _forward(gpu, 7, x.astype(np.float16), sel, w)
    want = G[f"moe_exact_{nt}"]
    _report(f"golden nt={nt}", got, want)
    assert np.array_equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [0.35, 0.05, 1.0])
def test_forward_sweep_bitexact(gpu, oracle, scale):
    """16 tokens x every expert of an 8-expert layer (128 picks, 16 slots per expert): exercises many rounding ties,
    small activations (fp16 subnormal range after the input Hadamard) and multi-pass slot chunks."""
    H, I, E = 512, 256, 8
    L = _layer(gpu, 5, E, H, I)
    ex = _host_experts(oracle, L)
    rng = np.random.default_rng(int(scale * 1000))
    x16 = (rng.standard_normal((16, H)) * scale).astype(np.float16)
    sel = np.tile(np.arange(E, dtype=np.int64), (16, 1))
    w = rng.random(sel.shape).astype(np.float32)
    got = _forward(gpu, 5, x16, sel, w)
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1)
    mx, rms, nbad = _report(f"sweep scale={scale}", got, want)
    assert nbad == 0


@pytest.mark.gpu
def test_forward_config0_single_expert(gpu, oracle):
    """Config 0: one routed expert H=5120 I=1536 K=3, M=1, weight 1."""
    H, I = 5120, 1536
    L = _layer(gpu, 2, 2, H, I)
    ex = _host_experts(oracle, L)
    rng = np.random.default_rng(5)
    x16 = rng.standard_normal((1, H)).astype(np.float16)
    sel = np.array([[1]], np.int64)
    w = np.ones((1, 1), np.float32)
    got = _forward(gpu, 2, x16, sel, w)
    want = oracle.expert_forward(ex[1], x16.astype(np.float32), mode=1)
    mx, rms, nbad = _report("config0", got, want)
    assert mx <= TOL * rms
    assert nbad == 0


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2])
def test_forward_layer_shape_bitexact(gpu, oracle, M):
    """Config-1 shape (H=5120, I=1536, K=3, top-8) on a 12-expert layer."""
    import synth
    H, I, E = 5120, 1536, 12
    L = _layer(gpu, 3, E, H, I)
    ex = _host_experts(oracle, L)
    rng = np.random.default_rng(100 + M)
    x16 = rng.standard_normal((M, H)).astype(np.float16)
    (sel, w16), _ = synth.route_uniform(M, E, 8, rng)
    got = _forward(gpu, 3, x16, sel, w16)
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w16.astype(np.float32), mode=1)
    mx, rms, nbad = _report(f"layer M={M}", got, want)
    assert mx <= TOL * rms
    assert nbad == 0


@pytest.mark.gpu
@pytest.mark.parametrize("Ks", [(4, 4, 3), (3, 3, 5), (2, 5, 4)])
def test_forward_mixed_k_bitexact(gpu, oracle, Ks):
    """Config-2 style mixed bitrates (K-generic decode in one kernel family), small shape."""
    H, I, E = 512, 256, 5
    L = _layer(gpu, 4, E, H, I, Ks)
    ex = _host_experts(oracle, L)
    rng = np.random.default_rng(sum(Ks))
    x16 = rng.standard_normal((3, H)).astype(np.float16)
    sel = np.array([[0, 2, 4], [1, 2, -1], [4, 3, 0]], np.int64)
    w = rng.random(sel.shape).astype(np.float32)
    got = _forward(gpu, 4, x16, sel, w)
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1)
    mx, rms, nbad = _report(f"mixed {Ks}", got, want)
    assert nbad == 0


@pytest.mark.gpu
def test_alignment_errors(gpu):
    """The gate|up input transform reads x and suh 16 bytes per lane: misaligned addresses are refused, not read."""
    import torch
    import _native
    L = _layer(gpu, 6, 2, 512, 256)
    bad = list(L.ptr_table)
    bad[3] += 2                       # suh_gate of expert 0, off its 16-byte alignment
    with pytest.raises(_native.NativeError, match="misaligned"):
        gpu.register_layer(7, 2, 512, 256, (3, 3, 3), bad)
    buf = torch.zeros(512 + 8, dtype=torch.float16, device="cuda")
    x = buf[1:513].view(1, 512)       # contiguous, 2 bytes off
    sel = torch.tensor([[0, 1]], dtype=torch.int64, device="cuda")
    w = torch.ones((1, 2), dtype=torch.float32, device="cuda")
    out = torch.empty((1, 512), dtype=torch.float32, device="cuda")
    with pytest.raises(_native.NativeError, match="16-byte aligned"):
        gpu.moe_forward(6, x, sel, w, out)


@pytest.mark.gpu
def test_empty_calls(gpu, oracle):
    """Empty calls as the reference's tier_forward takes them (ft_tier_ext.cpp:893-903): no tokens is a no-op, and
    tokens without picks (sel [M, 0]) give rows of zeros, which the oracle's moe_forward gives too; through the
    decode, no-allocation and grouped entry points, then a normal call on the same context still bit-exact."""
    import torch
    L = _layer(gpu, 8, 4, 512, 256)
    ex = _host_experts(oracle, L)
    f16 = dict(dtype=torch.float16, device="cuda")
    i64 = dict(dtype=torch.int64, device="cuda")
    f32 = dict(dtype=torch.float32, device="cuda")
    for fn in (gpu.moe_forward, gpu.moe_forward_noalloc, gpu.grouped_forward):
        name = fn.__name__
        print(f"empty calls: {name}", flush=True)
        out0 = torch.empty((0, 512), **f32)
        fn(8, torch.empty((0, 512), **f16), torch.empty((0, 8), **i64), torch.empty((0, 8), **f32), out0)
        x = torch.randn((3, 512), **f32).to(torch.float16)
        out = torch.full((3, 512), float("nan"), **f32)
        fn(8, x, torch.empty((3, 0), **i64), torch.empty((3, 0), **f32), out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        want = oracle.moe_forward(ex, x.float().cpu().numpy(), np.zeros((3, 0), np.int64), np.zeros((3, 0), np.float32),
                                  mode=1)
        assert np.array_equal(got, np.zeros((3, 512), np.float32)) and np.array_equal(want, got), name
        assert not np.signbit(got).any(), name
    rng = np.random.default_rng(800)
    x16 = rng.standard_normal((2, 512)).astype(np.float16)
    sel = np.array([[0, 1], [2, 3]], np.int64)
    w = rng.random((2, 2)).astype(np.float32)
    got = _forward(gpu, 8, x16, sel, w)
    _, _, nbad = _report("after empty calls", got, oracle.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1))
    assert nbad == 0


@pytest.mark.gpu
@pytest.mark.parametrize("ns", [1, 2, 4, 8])
def test_forward_slots_per_pass_bitexact(gpu, oracle, ns):
    """Every slots-per-pass instantiation (GFL_SLOTS_PER_PASS, read at context creation): 12 tokens over 6 experts, so
    experts hold up to 12 slots and take several passes over their weights."""
    import os
    import _native
    import synth
    old = os.environ.get("GFL_SLOTS_PER_PASS")
    os.environ["GFL_SLOTS_PER_PASS"] = str(ns)
    try:
        ctx = _native.Context(0)
    finally:
        if old is None:
            os.environ.pop("GFL_SLOTS_PER_PASS", None)
        else:
            os.environ["GFL_SLOTS_PER_PASS"] = old
    H, I, E = 512, 256, 6
    L = synth.SynthLayer(8, E, H, I, (3, 3, 3))
    L.register(ctx, 8)
    ex = _host_experts(oracle, L)
    rng = np.random.default_rng(100 + ns)
    M = 12
    x16 = rng.standard_normal((M, H)).astype(np.float16)
    sel = np.stack([rng.permutation(E)[:4] for _ in range(M)]).astype(np.int64)
    w = rng.random(sel.shape).astype(np.float32)
    got = _forward(ctx, 8, x16, sel, w)
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1)
    mx, rms, nbad = _report(f"slots per pass {ns}", got, want)
    assert nbad == 0


@pytest.mark.gpu
def test_forward_max_picks_bitexact(gpu, oracle):
    """The largest decode call: 128 tokens x top-8 = 1024 picks over 32 experts (every expert in several jobs)."""
    H, I, E = 512, 256, 32
    L = _layer(gpu, 9, E, H, I)
    ex = _host_experts(oracle, L)
    rng = np.random.default_rng(128)
    M = 128
    x16 = (rng.standard_normal((M, H)) * 0.5).astype(np.float16)
    sel = np.stack([rng.permutation(E)[:8] for _ in range(M)]).astype(np.int64)
    w = rng.random(sel.shape).astype(np.float32)
    got = _forward(gpu, 9, x16, sel, w)
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1)
    mx, rms, nbad = _report("max picks", got, want)
    assert nbad == 0


@pytest.mark.gpu
@pytest.mark.parametrize("w_half", [False, True])
def test_forward_duplicate_picks_bitexact(gpu, oracle, w_half):
    """A token may pick one expert twice (two slots, two weighted terms in job order); fp16 and fp32 weights."""
    H, I, E = 512, 256, 4
    L = _layer(gpu, 10, E, H, I)
    ex = _host_experts(oracle, L)
    rng = np.random.default_rng(11 + int(w_half))
    x16 = rng.standard_normal((3, H)).astype(np.float16)
    sel = np.array([[1, 1, 2], [3, 0, 3], [2, 2, 2]], np.int64)
    w = rng.random(sel.shape).astype(np.float16 if w_half else np.float32)
    got = _forward(gpu, 10, x16, sel, w, w_half=w_half)
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w.astype(np.float32), mode=1)
    mx, rms, nbad = _report(f"duplicate picks w_half={w_half}", got, want)
    assert nbad == 0


def _union_layer(gpu, li, sel, H, I, Ks):
    """A layer holding only the routed experts: ids are relabelled to their rank among the routed ones (job order
    depends on first appearance, not on the ids), and the layer's experts are synthetic like any other."""
    uniq = np.unique(sel[sel >= 0])
    remap = {int(e): i for i, e in enumerate(uniq)}
    sel2 = np.array([[remap[int(e)] if e >= 0 else -1 for e in row] for row in sel], np.int64)
    L = _layer(gpu, li, len(uniq), H, I, Ks)
    return L, sel2


@pytest.mark.gpu
@pytest.mark.parametrize("layer_kind", ["A_4_4_3", "B_3_3_5"])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_config2_full_shape_bitexact(gpu, oracle, layer_kind, M):
    """Config 2 at its shape: H=5120, I=1536, top-8 of 288 experts with Zipf-skewed (s=1.1) routing logits, layer A
    (gate/up 4 bpw, down 3) and layer B (gate/up 3, down 5); the K=4 and K=5 kernels at full size."""
    import synth
    Ks = {"A_4_4_3": (4, 4, 3), "B_3_3_5": (3, 3, 5)}[layer_kind]
    H, I, E = 5120, 1536, 288
    rng = np.random.default_rng(2000 + 10 * M + Ks[2])
    sel, w16 = synth.route(synth.zipf_logits(M, E, 1.1, rng), 8)
    L, sel2 = _union_layer(gpu, 20 + M, sel, H, I, Ks)
    ex = _host_experts(oracle, L)
    x16 = rng.standard_normal((M, H)).astype(np.float16)
    got = _forward(gpu, 20 + M, x16, sel2, w16)
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel2, w16.astype(np.float32), mode=1)
    mx, rms, nbad = _report(f"config2 {layer_kind} M={M} union={L.E}", got, want)
    assert mx <= TOL * rms
    assert nbad == 0


@pytest.mark.gpu
@pytest.mark.parametrize("M", [16, 32, 64])
def test_config3_full_shape_bitexact(gpu, oracle, M):
    """Config 3 at its shape: M = 16, 32 and 64 tokens, each routed top-8 over 288 experts with uniform N(0,1) logits,
    H=5120, I=1536, 3 bpw, through the default launch choice (above 8 tokens: a workgroup per routed expert taking
    its slots two per pass, gu_kernel / down_kernel with NS = 2). The layer holds the routed union (up to 240
    experts, 2.1 GB); the oracle evaluates rows 0, M/2 and M-1 with the whole call's jobs (moe_forward_rows), so each
    checked row's combine order is the full batch's."""
    import synth
    from oracle import Mat
    H, I, E = 5120, 1536, 288
    rng = np.random.default_rng(3000 + M)
    (sel, w16), _ = synth.route_uniform(M, E, 8, rng)
    L, sel2 = _union_layer(gpu, 40 + M, sel, H, I, (3, 3, 3))
    x16 = rng.standard_normal((M, H)).astype(np.float16)
    got = _forward(gpu, 40 + M, x16, sel2, w16)
    rows = [0, M // 2, M - 1]
    need = {int(e) for r in rows for e in sel2[r] if e >= 0}
    dummy = None
    ex = []
    for e in range(L.E):
        if e in need or dummy is None:
            mats = []
            for p in range(3):
                tr, suh, svh = L.matrix(e, p)
                k, n = (H, I) if p < 2 else (I, H)
                mats.append(Mat(tr, suh, svh, k, n, 3))
            ex.append(tuple(mats))
            if dummy is None:
                dummy = ex[-1]
        else:
            ex.append(dummy)       # never read: no checked row picks it
    want = oracle.moe_forward_rows(ex, x16.astype(np.float32), sel2, w16.astype(np.float32), rows, mode=1)
    mx, rms, nbad = _report(f"config3 M={M} union={L.E} rows {rows}", got[rows], want)
    assert mx <= TOL * rms
    assert nbad == 0
    assert np.all(np.isfinite(got)) and float(np.sqrt(np.mean(got.astype(np.float64) ** 2))) > 0


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [1, 0, 2, -1])
def test_every_mode_number_computes_exact(gpu, oracle, mode):
    """tier_forward's mode numbers (-1 auto, 0 AFFINE, 1 EXACT, 2 I16; ft_tier_ext.cpp:865-904) all compute EXACT
    on the device, bit-identical to the reference's EXACT mode."""
    import torch
    H, I, E = 512, 256, 6
    L = _layer(gpu, 30, E, H, I)
    ex = _host_experts(oracle, L)
    rng = np.random.default_rng(31)
    x16 = rng.standard_normal((2, H)).astype(np.float16)
    sel = np.array([[0, 3, 5], [2, 3, -1]], np.int64)
    w = rng.random(sel.shape).astype(np.float32)
    xd = torch.from_numpy(x16.view(np.int16)).view(torch.float16).cuda()
    out = torch.empty((2, H), dtype=torch.float32, device="cuda")
    gpu.moe_forward(30, xd, torch.from_numpy(sel).cuda(), torch.from_numpy(w).cuda(), out, mode=mode)
    torch.cuda.synchronize()
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1)
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.gpu
def test_width_mismatch_is_refused(gpu):
    """x / out narrower or wider than the layer's H are refused before any launch (the C ABI takes no H)."""
    import torch
    _layer(gpu, 31, 2, 512, 256)
    assert gpu.layer_info(31) == (2, 512, 256, 3, 3, 3)
    sel = torch.tensor([[0, 1]], dtype=torch.int64, device="cuda")
    w = torch.ones((1, 2), dtype=torch.float32, device="cuda")
    for width in (256, 768):
        x = torch.zeros((1, width), dtype=torch.float16, device="cuda")
        out = torch.empty((1, width), dtype=torch.float32, device="cuda")
        with pytest.raises(ValueError, match="H = 512"):
            gpu.moe_forward(31, x, sel, w, out)
        with pytest.raises(ValueError, match="H = 512"):
            gpu.grouped_forward(31, x, sel, w, out)


@pytest.mark.gpu
def test_graph_replay_after_a_larger_eager_call(gpu, oracle):
    """A graph captured at M=1 keeps working after an eager M=128 call (workspaces are reserved, never freed while
    the context lives): every replay matches the eager M=1 result."""
    import torch
    H, I, E = 512, 256, 16
    L = _layer(gpu, 32, E, H, I)
    ex = _host_experts(oracle, L)
    rng = np.random.default_rng(32)
    x1 = rng.standard_normal((1, H)).astype(np.float16)
    sel1 = np.array([[3, 7, 1, 9, 0, 15, 4, 8]], np.int64)
    w1 = rng.random(sel1.shape).astype(np.float32)
    xd = torch.from_numpy(x1.view(np.int16)).view(torch.float16).cuda()
    sd, wd = torch.from_numpy(sel1).cuda(), torch.from_numpy(w1).cuda()
    out = torch.empty((1, H), dtype=torch.float32, device="cuda")
    gpu.moe_forward(32, xd, sd, wd, out)
    torch.cuda.synchronize()
    want1 = oracle.moe_forward(ex, x1.astype(np.float32), sel1, w1, mode=1)
    assert np.array_equal(out.cpu().numpy(), want1)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            gpu.moe_forward(32, xd, sd, wd, out)
    torch.cuda.current_stream().wait_stream(st)
    M = 128
    xb = rng.standard_normal((M, H)).astype(np.float16)
    selb = np.stack([rng.permutation(E)[:8] for _ in range(M)]).astype(np.int64)
    wb = rng.random(selb.shape).astype(np.float32)
    for rep in range(3):
        outb = torch.empty((M, H), dtype=torch.float32, device="cuda")
        gpu.moe_forward(32, torch.from_numpy(xb.view(np.int16)).view(torch.float16).cuda(),
                        torch.from_numpy(selb).cuda(), torch.from_numpy(wb).cuda(), outb)
        torch.cuda.synchronize()
        if rep == 0:
            wantb = oracle.moe_forward(ex, xb.astype(np.float32), selb, wb, mode=1)
            assert np.array_equal(outb.cpu().numpy(), wantb)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), want1), f"replay {rep}"


@pytest.mark.gpu
def test_against_both_reference_builds(gpu, oracle, ref, ref_server):
    """Config-1 width (H=5120, I=1536, K=3), 8 experts, 4 tokens x top-4 with a skipped pick: bit-exact against the
    reference engine's A/B build (-ffp-contract=off); against its server build (default contraction) the max-abs is
    reported and held to the north-star 2e-3 * RMS."""
    H, I, E = 5120, 1536, 8
    L = _layer(gpu, 12, E, H, I)
    ex = _host_experts(oracle, L)
    rng = np.random.default_rng(1212)
    x16 = rng.standard_normal((4, H)).astype(np.float16)
    sel = np.stack([rng.permutation(E)[:4] for _ in range(4)]).astype(np.int64)
    sel[2, 1] = -1
    w = rng.random(sel.shape).astype(np.float32)
    got = _forward(gpu, 12, x16, sel, w)
    a = ref.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1)
    b = ref_server.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1)
    _report("vs A/B build", got, a)
    mx, rms, _ = _report("vs server build", got, b)
    assert np.array_equal(got, a)
    assert mx <= TOL * rms


def _ctx_with_env(**env):
    """A context created under the given environment (read once at creation: GFL_RELAY, GFL_STREAM, ...)."""
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


def _relay_env(relay, prio):
    return dict(GFL_RELAY=relay, **({"GFL_RELAY_PRIO": prio} if prio else {}))


@pytest.mark.gpu
@pytest.mark.parametrize("prio", [None, "1,1"])
@pytest.mark.parametrize("relay", ["0", "1,1", "2,2", "4,4", "2,1", "4,2", "1,4"])
def test_relay_launches_bitexact(gpu, oracle, relay, prio):
    """Every decode launch family of one slot per pass (GFL_RELAY, read at context creation): without relay ("0"), and
    the relay launches with 1, 2 or 4 waves per tile column for gate|up and down; mixed K (2..5), skipped picks, a token
    picking one expert twice, and 1, 2 and 5 tokens. With prio "1,1" (GFL_RELAY_PRIO) the relay waves lower their issue
    priority as they progress, which these small launches would not choose by themselves."""
    ctx = _ctx_with_env(**_relay_env(relay, prio))
    H, I = 512, 256
    for li, Ks in enumerate([(3, 3, 3), (2, 5, 4), (4, 4, 3), (5, 2, 5)]):
        L = _layer(ctx, 40 + li, 6, H, I, Ks)
        ex = _host_experts(oracle, L)
        for M in (1, 2, 5):
            rng = np.random.default_rng(4000 + 10 * li + M)
            x16 = rng.standard_normal((M, H)).astype(np.float16)
            sel = np.stack([rng.permutation(6)[:4] for _ in range(M)]).astype(np.int64)
            if M >= 2:
                sel[1, 2] = -1
                sel[0, 3] = sel[0, 0]
            w = rng.random(sel.shape).astype(np.float32)
            got = _forward(ctx, 40 + li, x16, sel, w)
            want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1)
            _, _, nbad = _report(f"relay {relay} Ks {Ks} M={M}", got, want)
            assert nbad == 0


@pytest.mark.gpu
@pytest.mark.parametrize("relay,prio", [("4,4", None), ("2,1", None), ("2,1", "0,0"), ("2,2", None), ("1,1", None),
                                        ("1,1", "1,1")])
def test_relay_launches_full_shape_bitexact(gpu, oracle, relay, prio):
    """The relay launches at the config-1 shape (H=5120, I=1536, K=3): one expert (config 0) and top-8 of a
    10-expert layer at M = 1 and 3; the progress priority as each launch chooses it (on at M = 1 for "2,1"), or forced
    off / on (GFL_RELAY_PRIO)."""
    import synth
    ctx = _ctx_with_env(**_relay_env(relay, prio))
    H, I, E = 5120, 1536, 10
    L = _layer(ctx, 50, E, H, I)
    ex = _host_experts(oracle, L)
    rng = np.random.default_rng(5000)
    x16 = rng.standard_normal((1, H)).astype(np.float16)
    sel = np.array([[7]], np.int64)
    got = _forward(ctx, 50, x16, sel, np.ones((1, 1), np.float32))
    want = oracle.expert_forward(ex[7], x16.astype(np.float32), mode=1)
    _, _, nbad = _report(f"relay {relay} one expert", got, want)
    assert nbad == 0
    for M in (1, 3):
        rng = np.random.default_rng(5000 + M)
        x16 = rng.standard_normal((M, H)).astype(np.float16)
        (sel, w16), _ = synth.route_uniform(M, E, 8, rng)
        got = _forward(ctx, 50, x16, sel, w16)
        want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w16.astype(np.float32), mode=1)
        mx, rms, nbad = _report(f"relay {relay} full shape M={M}", got, want)
        assert mx <= TOL * rms
        assert nbad == 0


@pytest.mark.gpu
@pytest.mark.parametrize("relay", [None, "1,1"])
def test_one_slot_per_pass_above_64_picks_bitexact(gpu, oracle, relay):
    """Top-16 at M = 5 and 8 (80 and 128 picks, one slot per pass): more picks than the relay down launch's combine
    list holds (one per lane of a wave), so these calls keep the per-slot launches, under the default launch choice
    and with the relay forced (GFL_RELAY applies up to 64 picks); every token's row bit-exact, including tokens past
    the first 64 picks. At 64 picks (M = 4) the relay launches run."""
    ctx = gpu if relay is None else _ctx_with_env(GFL_RELAY=relay)
    H, I, E, li = 512, 256, 20, 54 if relay is None else 55
    L = _layer(ctx, li, E, H, I, (3, 4, 3))
    ex = _host_experts(oracle, L)
    for M in (4, 5, 8):
        rng = np.random.default_rng(5400 + M)
        x16 = rng.standard_normal((M, H)).astype(np.float16)
        sel = np.stack([rng.permutation(E)[:16] for _ in range(M)]).astype(np.int64)
        sel[M - 1, 3] = -1
        w = rng.random(sel.shape).astype(np.float32)
        got = _forward(ctx, li, x16, sel, w)
        want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1)
        _, _, nbad = _report(f"relay {relay} top-16 M={M}", got, want)
        assert nbad == 0


@pytest.mark.gpu
def test_shared_context_launch_choice_bitexact(gpu, oracle):
    """At 8 picks of the config-1 shape the default context runs the relay launches and a context told that other GPU
    work runs beside it (gfl_ctx_set_shared) keeps the per-slot launches: both bit-exact against the oracle, on the
    same inputs, and the flag can be switched between calls."""
    import synth
    import _native
    ctx = _native.Context(0)
    H, I, E = 5120, 1536, 10
    L = _layer(ctx, 52, E, H, I)
    ex = _host_experts(oracle, L)
    rng = np.random.default_rng(5200)
    x16 = rng.standard_normal((1, H)).astype(np.float16)
    (sel, w16), _ = synth.route_uniform(1, E, 8, rng)
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w16.astype(np.float32), mode=1)
    for shared in (False, True, False):
        ctx.set_shared(shared)
        got = _forward(ctx, 52, x16, sel, w16)
        _, _, nbad = _report(f"shared={shared} 8 picks", got, want)
        assert nbad == 0
    ctx.set_shared(False)
