"""Prefill path (gfl_grouped_forward: MFMA grouped GEMMs, an explicit opt-in outside the north-star bar) against the
reference's EXACT mode and its fp64 expert.

The grouped path keeps the bit-exact fp16 weights and every fp16 rounding point of the reference's transforms but
forms the hidden-dimension sums in MFMA order, so it differs from EXACT by fp32 accumulation rounding, about as far as
the reference's own fp64 expert (ref_expert) lies from EXACT on config-0 experts (max-abs 2.9e-3..3.3e-3 of the output
RMS). It misses the 2e-3 max-abs bar that EXACT meets, so no reference mode number routes to it (tier_forward and
gfl_moe_forward compute EXACT at every size). Bars, set to what the path measures on these cases (max-abs 1.5e-3 to
3.6e-3 of the output RMS, rel-RMS 1.6e-4 to 3.6e-4; config 4: 2.93e-3 and 3.6e-4):
  * RMS of the difference <= 5e-4 of the output RMS;
  * max-abs difference <= 4e-3 of the output RMS;
  * for one expert, the distance to the fp64 reference is within 2x of EXACT's own distance to it.
"""
import numpy as np
import pytest

REL_RMS = 5e-4
MAX_ABS = 4e-3


def _layer(gpu, li, E, H, I, Ks=(3, 3, 3)):
    import synth
    L = synth.SynthLayer(li, E, H, I, Ks)
    L.register(gpu, li)
    return L


def _host_experts(L):
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


def _run(gpu, li, x16, sel, w, grouped=True):
    import torch
    xd = torch.from_numpy(x16.view(np.int16)).view(torch.float16).cuda()
    seld = torch.from_numpy(np.ascontiguousarray(sel, dtype=np.int64)).cuda()
    wd = torch.from_numpy(np.ascontiguousarray(w)).cuda()
    out = torch.full(x16.shape, float("nan"), dtype=torch.float32, device="cuda")
    if grouped:
        gpu.grouped_forward(li, xd.contiguous(), seld, wd, out)
    else:
        gpu.moe_forward(li, xd.contiguous(), seld, wd, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _stats(name, got, want):
    d = got.astype(np.float64) - want.astype(np.float64)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    rel = float(np.sqrt(np.mean(d ** 2))) / rms
    mx = float(np.abs(d).max()) / rms
    print(f"{name}: rms {rms:.3e} rel-rms {rel:.2e} max-abs/rms {mx:.2e} bit-equal {np.mean(got == want):.3f}")
    return rel, mx


@pytest.mark.gpu
@pytest.mark.parametrize("M,topk", [(64, 4), (200, 8), (1, 8)])
def test_grouped_small_vs_exact(gpu, oracle, M, topk):
    """Random routing with skipped picks (-1) on an 8-expert layer; several passes of 64 slots per expert at M=200."""
    H, I, E = 512, 256, 8
    L = _layer(gpu, 21, E, H, I)
    ex = _host_experts(L)
    rng = np.random.default_rng(M * 31 + topk)
    x16 = rng.standard_normal((M, H)).astype(np.float16)
    sel = np.stack([rng.permutation(E)[:topk] for _ in range(M)]).astype(np.int64)
    sel[rng.random(sel.shape) < 0.1] = -1
    w = rng.random(sel.shape).astype(np.float32)
    w[sel < 0] = 0.0
    got = _run(gpu, 21, x16, sel, w)
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1)
    assert np.isfinite(got).all()
    rel, mx = _stats(f"grouped M={M} top{topk}", got, want)
    assert rel <= REL_RMS and mx <= MAX_ABS


@pytest.mark.gpu
def test_grouped_token_without_picks_is_zero(gpu):
    H, I, E = 512, 256, 4
    _layer(gpu, 22, E, H, I)
    rng = np.random.default_rng(9)
    x16 = rng.standard_normal((3, H)).astype(np.float16)
    sel = np.array([[0, 1], [-1, -1], [2, 3]], np.int64)
    w = np.array([[0.5, 0.5], [0.0, 0.0], [0.25, 0.75]], np.float32)
    got = _run(gpu, 22, x16, sel, w)
    assert np.all(got[1] == 0.0)
    assert np.isfinite(got).all() and np.abs(got[0]).max() > 0


@pytest.mark.gpu
@pytest.mark.parametrize("Ks", [(4, 4, 3), (3, 3, 5), (2, 5, 4)])
def test_grouped_mixed_k(gpu, oracle, Ks):
    """Config-2 style mixed bitrates, including gate and up at different K (two gate|up launches)."""
    H, I, E = 512, 256, 5
    L = _layer(gpu, 23, E, H, I, Ks)
    ex = _host_experts(L)
    rng = np.random.default_rng(sum(Ks))
    M = 96
    x16 = rng.standard_normal((M, H)).astype(np.float16)
    sel = np.stack([rng.permutation(E)[:3] for _ in range(M)]).astype(np.int64)
    w = rng.random(sel.shape).astype(np.float32)
    got = _run(gpu, 23, x16, sel, w)
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1)
    rel, mx = _stats(f"grouped mixed {Ks}", got, want)
    assert rel <= REL_RMS and mx <= MAX_ABS


@pytest.mark.gpu
def test_grouped_config_shape_vs_decode_path(gpu):
    """Config-1 shape (H=5120, I=1536, K=3, top-8 of 288), M=128: against the bit-exact decode path on the GPU."""
    import synth
    H, I, E = 5120, 1536, 288
    _layer(gpu, 24, E, H, I)
    rng = np.random.default_rng(24)
    M = 128
    x16 = rng.standard_normal((M, H)).astype(np.float16)
    (sel, w16), _ = synth.route_uniform(M, E, 8, rng)
    exact = _run(gpu, 24, x16, sel, w16, grouped=False)
    got = _run(gpu, 24, x16, sel, w16)
    rel, mx = _stats("grouped config1 M=128", got, exact)
    assert rel <= REL_RMS and mx <= MAX_ABS


@pytest.mark.gpu
def test_grouped_single_expert_vs_fp64(gpu, oracle):
    """Config 0 (one expert, H=5120 I=1536 K=3): the grouped result is about as close to the reference's fp64 expert
    as the reference's EXACT mode is."""
    H, I = 5120, 1536
    L = _layer(gpu, 25, 2, H, I)
    ex = _host_experts(L)
    rng = np.random.default_rng(25)
    x16 = rng.standard_normal((1, H)).astype(np.float16)
    sel = np.array([[1]], np.int64)
    w = np.ones((1, 1), np.float32)
    got = _run(gpu, 25, x16, sel, w)[0]
    exact = oracle.expert_forward(ex[1], x16.astype(np.float32), mode=1)[0]
    r64 = oracle.expert_ref64(ex[1], x16[0].astype(np.float32))
    rel_g, mx_g = _stats("grouped vs fp64", got, r64)
    rel_e, mx_e = _stats("EXACT vs fp64", exact, r64)
    _stats("grouped vs EXACT", got, exact)
    assert rel_g <= 2 * rel_e + 1e-5
    assert mx_g <= 2 * mx_e + 1e-5


@pytest.mark.gpu
def test_grouped_duplicate_picks(gpu, oracle):
    """Tokens that pick one expert twice, through the grouped path (fp16 weights)."""
    H, I, E = 512, 256, 4
    L = _layer(gpu, 26, E, H, I)
    ex = _host_experts(L)
    rng = np.random.default_rng(26)
    M = 40
    x16 = rng.standard_normal((M, H)).astype(np.float16)
    sel = rng.integers(0, E, size=(M, 3)).astype(np.int64)       # duplicates within a token are common
    w = rng.random(sel.shape).astype(np.float16)
    got = _run(gpu, 26, x16, sel, w)
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w.astype(np.float32), mode=1)
    rel, mx = _stats("grouped duplicates", got, want)
    assert rel <= REL_RMS and mx <= MAX_ABS


def _routing(mode, M, topk, E, rng):
    """Routings for the plan test: distinct experts per token (uniform), Zipf-skewed picks with repeats within a token
    (skew, dups), and skipped (-1) and out-of-range ids sprinkled in (bad)."""
    if mode == "uniform":
        return np.stack([rng.permutation(E)[:topk] for _ in range(M)]).astype(np.int64)
    p = 1.0 / np.arange(1, E + 1) ** (1.3 if mode == "skew" else 0.6)
    sel = rng.choice(E, size=(M, topk), p=p / p.sum()).astype(np.int64)
    if mode == "bad":
        m = rng.random(sel.shape)
        sel[m < 0.1] = -1
        sel[(m >= 0.1) & (m < 0.13)] = E + rng.integers(0, 5)
        sel[(m >= 0.13) & (m < 0.15)] = -7
    return sel


@pytest.mark.gpu
@pytest.mark.parametrize("M,topk,E,mode", [(2048, 8, 288, "uniform"), (1500, 6, 64, "skew"), (3000, 8, 16, "dups"),
                                           (333, 16, 1024, "bad"), (4096, 16, 40, "bad")])
def test_grouped_plan_is_the_reference_order(gpu, oracle, M, topk, E, mode):
    """The device plan of the grouped path over several chunks of 1024 picks, exactly: expert-major slots with picks
    ascending (tier_lut_build_grouped_rows), and each token's picks in the order of the reference's jobs
    (moe_forward's token-major scan, a new job every 8 picks of an expert; the oracle's build_jobs)."""
    import torch
    rng = np.random.default_rng(M * 7 + topk + E)
    sel = _routing(mode, M, topk, E, rng)
    w = rng.standard_normal(sel.shape).astype(np.float16)
    r = gpu.grouped_plan(torch.from_numpy(sel).cuda(), torch.from_numpy(w.view(np.int16)).view(torch.float16).cuda(), E)
    torch.cuda.synchronize()
    r = {k: v.cpu().numpy() for k, v in r.items()}
    P = M * topk
    flat = sel.reshape(-1)
    valid = (flat >= 0) & (flat < E)
    S = int(valid.sum())
    assert r["hdr"].tolist() == [S, int(((flat != -1) & ~valid).sum())]
    cnt = np.bincount(flat[valid], minlength=E)
    assert np.array_equal(r["off"], np.concatenate([[0], np.cumsum(cnt)]))
    picks = np.nonzero(valid)[0]
    order = np.lexsort((picks, flat[picks]))
    assert np.array_equal(r["slot_pick"][:S], picks[order])
    assert np.array_equal(r["slot_e"][:S], flat[picks][order])
    slot_of = np.full(P, -1, np.int64)
    slot_of[picks[order]] = np.arange(S)
    # job of every valid pick from the oracle's job list: the c-th pick (scan order) of expert e sits at entry c % 8
    # of e's (c // 8)-th job
    sel_o = np.where((sel >= 0) & (sel < E), sel, -1)
    jobs = oracle.build_jobs(E, sel_o, w.astype(np.float32))
    of_e = {}
    for j, (e, members) in enumerate(jobs):
        of_e.setdefault(e, []).append(j)
    job = np.full(P, -1, np.int64)
    seen = np.zeros(E, np.int64)
    for p in picks:
        e, t = int(flat[p]), p // topk
        c = seen[e]
        seen[e] += 1
        j = of_e[e][c // 8]
        assert jobs[j][1][c % 8] == (t, float(w.reshape(-1)[p]))
        job[p] = j
    npk = valid.reshape(M, topk).sum(1)
    assert np.array_equal(r["tok_npk"], npk)
    for t in range(M):
        ks = [k for k in range(topk) if valid[t * topk + k]]
        ks.sort(key=lambda k: (job[t * topk + k], k))
        assert r["tok_slot"][t, :len(ks)].tolist() == [int(slot_of[t * topk + k]) for k in ks], t
        assert np.array_equal(r["tok_w"][t, :len(ks)], np.array([w[t, k] for k in ks], np.float32)), t


@pytest.mark.gpu
def test_config4_prefill_exact_rows_and_grouped_vs_exact(gpu, oracle):
    """Config 4 prefill: M=2048 tokens, top-8 of 288 experts, H=5120 I=1536 K=3 (16,384 picks).
    EXACT (gfl_moe_forward above 1024 picks): four tokens' rows bit-exact against the oracle's layer forward with the
    whole batch's jobs (each token's combine order is the full call's). Grouped MFMA path: all 2048 rows against that
    EXACT result, with max-abs/RMS and the count of elements beyond the north-star 2e-3 * RMS reported, and the
    path's bars asserted."""
    import synth
    from oracle import Mat
    H, I, E, M = 5120, 1536, 288, 2048
    L = _layer(gpu, 25, E, H, I)
    rng = np.random.default_rng(5000 + 2048)
    x16 = rng.standard_normal((M, H)).astype(np.float16)
    (sel, w16), _ = synth.route_uniform(M, E, 8, rng)
    print("config4: EXACT M=2048", flush=True)
    exact = _run(gpu, 25, x16, sel, w16, grouped=False)
    print("config4: grouped M=2048", flush=True)
    grouped = _run(gpu, 25, x16, sel, w16)
    assert np.isfinite(exact).all() and np.isfinite(grouped).all()
    rows = [0, 777, 1500, 2047]
    need = sorted(set(int(e) for r in rows for e in sel[r]))
    mats = {}
    for e in need:
        ms = []
        for p in range(3):
            tr, suh, svh = L.matrix(e, p)
            k, n = (H, I) if p < 2 else (I, H)
            ms.append(Mat(tr, suh, svh, k, n, 3))
        mats[e] = tuple(ms)
    ex = [mats.get(e, mats[need[0]]) for e in range(E)]   # experts no wanted row picks are never read
    want = oracle.moe_forward_rows(ex, x16.astype(np.float32), sel, w16.astype(np.float32), rows, mode=1)
    nbad = int(np.count_nonzero(exact[rows] != want))
    print(f"config4 EXACT rows {rows}: mismatched {nbad}/{want.size}")
    assert nbad == 0
    rel, mx = _stats("config4 grouped vs EXACT, all 2048 rows", grouped, exact)
    rms = float(np.sqrt(np.mean(exact.astype(np.float64) ** 2)))
    beyond = int(np.count_nonzero(np.abs(grouped.astype(np.float64) - exact) > 2e-3 * rms))
    print(f"config4 grouped: elements beyond 2e-3*RMS: {beyond}/{exact.size}")
    assert rel <= REL_RMS and mx <= MAX_ABS