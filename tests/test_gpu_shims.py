"""The reference-shaped surface on the GPU: a full-residency expert_cache.Pool over duck-typed MoE modules, the tier
registered from it as cpu_tier.start does, tier_forward (the reference's expert-call signature: CPU fp32 x, int32 sel
with -1 skips, fp32 w) bit-identical to the oracle, the SwiGLU clamp through tier_set_act_limit, and the split through
the handle k_ftsplit.install swaps in."""
import numpy as np
import pytest
import torch

import fake_moe

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tier(gpu):
    import expert_cache
    import ft_tier
    import synth
    H, I, E = 512, 256, 6
    layers = [synth.SynthLayer(40 + li, E, H, I, Ks) for li, Ks in enumerate(((3, 3, 3), (4, 4, 3)))]
    mods = [fake_moe.from_synth(L, f"model.layers.{li}.mlp") for li, L in enumerate(layers)]
    pool = expert_cache.Pool(torch.device("cuda", 0), mods)
    ft_tier.tier_shutdown()
    ctrl = torch.zeros(16, dtype=torch.int64, device="cuda")
    hx = torch.zeros(4 * H, dtype=torch.float16, device="cuda")
    picks = torch.zeros(4 * 8 * 3, dtype=torch.int32, device="cuda")
    hout = torch.zeros(4 * H, dtype=torch.float32, device="cuda")
    ft_tier.tier_init(1, [0], ctrl, hx, picks, hout, -1, H, I, len(mods), 0)
    ft_tier.add_pool_layers(pool, bits=[L.Ks for L in layers])
    yield dict(pool=pool, layers=layers, mods=mods, H=H, I=I, E=E, ctrl=ctrl, hx=hx, picks=picks, hout=hout)
    ft_tier.tier_set_act_limit(0.0)
    ft_tier.tier_shutdown()


def _experts(oracle, L):
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


@pytest.mark.parametrize("li", [0, 1])
def test_tier_forward_reference_signature_bitexact(tier, oracle, li):
    import ft_tier
    rng = np.random.default_rng(50 + li)
    m = 5
    x = torch.from_numpy((rng.standard_normal((m, tier["H"])) * 0.4).astype(np.float16).astype(np.float32))
    sel = torch.from_numpy(np.stack([rng.choice(tier["E"], 4, replace=False) for _ in range(m)]).astype(np.int32))
    sel[1, 2] = -1
    w = torch.from_numpy(rng.random((m, 4)).astype(np.float32))
    got = ft_tier.tier_forward(li, x, sel, w, -1)
    assert got.device.type == "cpu" and got.dtype == torch.float32 and tuple(got.shape) == (m, tier["H"])
    want = oracle.moe_forward(_experts(oracle, tier["layers"][li]), x.numpy(), sel.numpy(), w.numpy(), mode=1)
    assert np.array_equal(got.numpy(), want)
    st = ft_tier.tier_stats()
    assert len(st) == 12 and st[0] >= 1


@pytest.mark.parametrize("mode", [-1, 0, 2])
def test_tier_forward_prefill_sizes_every_mode_exact(tier, oracle, mode):
    """m * k > 1024 in the reference's auto, AFFINE and I16 modes: the EXACT layer, bit for bit (one policy for every
    mode number at every size, as gfl_moe_forward; the MFMA grouped path is only reached through
    gfl_grouped_forward)."""
    import ft_tier
    rng = np.random.default_rng(70 + mode)
    m = 300
    x = torch.from_numpy((rng.standard_normal((m, tier["H"])) * 0.5).astype(np.float16).astype(np.float32))
    sel = torch.from_numpy(np.stack([rng.choice(tier["E"], 4, replace=False) for _ in range(m)]).astype(np.int32))
    sel[7, 1] = -1
    w = torch.from_numpy(rng.random((m, 4)).astype(np.float32))
    got = ft_tier.tier_forward(1, x, sel, w, mode).numpy()
    want = oracle.moe_forward(_experts(oracle, tier["layers"][1]), x.numpy(), sel.numpy(), w.numpy(), mode=1)
    assert np.array_equal(got, want)


def test_tier_forward_exact_prefill_bitexact(tier, oracle):
    """m * k > 1024 in EXACT mode (1): bit-identical to the oracle's EXACT layer, as the reference's EXACT mode is at
    any batch size."""
    import ft_tier
    rng = np.random.default_rng(71)
    m = 300
    x = torch.from_numpy((rng.standard_normal((m, tier["H"])) * 0.5).astype(np.float16).astype(np.float32))
    sel = torch.from_numpy(np.stack([rng.choice(tier["E"], 4, replace=False) for _ in range(m)]).astype(np.int32))
    sel[9, 0] = -1
    w = torch.from_numpy(rng.random((m, 4)).astype(np.float32))
    got = ft_tier.tier_forward(1, x, sel, w, 1).numpy()
    want = oracle.moe_forward(_experts(oracle, tier["layers"][1]), x.numpy(), sel.numpy(), w.numpy(), mode=1)
    assert np.array_equal(got, want)


def test_tier_selftest_mode_loop(tier, oracle):
    """The reference's start-up self-test calls tier_forward(li, x, sel, w, mode) for mode in (1, 0, 2)
    (glm53/cpu_tier.py:766-773): every mode returns the EXACT layer."""
    import ft_tier
    rng = np.random.default_rng(77)
    x = torch.from_numpy((rng.standard_normal((2, tier["H"])) * 0.5).astype(np.float16).astype(np.float32))
    sel = torch.tensor([[0, 3, 1, 5], [2, 4, 0, -1]], dtype=torch.int32)
    w = torch.from_numpy(rng.random((2, 4)).astype(np.float32))
    want = oracle.moe_forward(_experts(oracle, tier["layers"][0]), x.numpy(), sel.numpy(), w.numpy(), mode=1)
    for mode in (1, 0, 2):
        assert np.array_equal(ft_tier.tier_forward(0, x, sel, w, mode).numpy(), want), mode


def test_tier_forward_act_limit(tier, oracle):
    import ft_tier
    rng = np.random.default_rng(60)
    x = torch.from_numpy((rng.standard_normal((3, tier["H"])) * 0.8).astype(np.float16).astype(np.float32))
    sel = torch.tensor([[0, 1, 2, 3], [2, 3, 4, 5], [5, 0, 1, 4]], dtype=torch.int32)
    w = torch.full((3, 4), 0.25)
    lim = 0.05
    ft_tier.tier_set_act_limit(lim)
    try:
        got = ft_tier.tier_forward(0, x, sel, w, 1)
    finally:
        ft_tier.tier_set_act_limit(0.0)
    ex = _experts(oracle, tier["layers"][0])
    want = oracle.moe_forward(ex, x.numpy(), sel.numpy(), w.numpy(), mode=1, act_limit=lim)
    free = oracle.moe_forward(ex, x.numpy(), sel.numpy(), w.numpy(), mode=1)
    assert not np.array_equal(want, free)           # the clamp is active at this limit
    assert np.array_equal(got.numpy(), want)


def test_tier_forward_argument_errors(tier):
    import ft_tier
    x = torch.full((1, tier["H"]), 0.1)              # 0.1 is not an fp16 value
    sel = torch.zeros(1, 4, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="fp16-valued"):
        ft_tier.tier_forward(0, x, sel, torch.ones(1, 4), 1)
    with pytest.raises(RuntimeError, match="mode must be"):
        ft_tier.tier_forward(0, x.half().float(), sel, torch.ones(1, 4), 3)
    with pytest.raises(RuntimeError, match="out of range"):
        ft_tier.tier_forward(0, x.half().float(), sel + 99, torch.ones(1, 4), 1)
    with pytest.raises(RuntimeError, match="already initialised"):
        e = torch.empty(0)
        ft_tier.tier_init(1, [0], e, e, e, e, -1, tier["H"], tier["I"], 1, 0)


def test_tier_forward_empty_calls(tier):
    """m = 0 returns an empty [0, H] result and sel [m, 0] rows of zeros, as the reference's tier_forward builds them
    (torch::zeros of [m, H], ft_tier_ext.cpp:893-903)."""
    import ft_tier
    H = tier["H"]
    out = ft_tier.tier_forward(0, torch.zeros(0, H), torch.zeros(0, 4, dtype=torch.int32), torch.zeros(0, 4), 1)
    assert tuple(out.shape) == (0, H) and out.dtype == torch.float32 and not out.is_cuda
    x = torch.randn(2, H).half().float()
    out = ft_tier.tier_forward(0, x, torch.zeros(2, 0, dtype=torch.int32), torch.zeros(2, 0), -1)
    assert tuple(out.shape) == (2, H) and torch.equal(out, torch.zeros(2, H))
    out = ft_tier.tier_forward(0, x.cuda(), torch.zeros(2, 0, dtype=torch.int32), torch.zeros(2, 0), 1)
    assert out.is_cuda and torch.equal(out.cpu(), torch.zeros(2, H))


def test_pool_on_device_verifies_clean(tier):
    r = tier["pool"].verify()
    assert r["bad_slots"] == 0 and r["bad_tables"] == 0 and r["owned"] == 2 * tier["E"]
    tier["pool"].step(0, torch.tensor([[0, 1, 2, 3]], device="cuda"), True)
    assert tier["pool"].summary()["hits"] >= 4


def test_installed_split_handle_on_device(tier, oracle):
    """cpu_tier.routed's call, through the handle k_ftsplit.install puts in place, with the pool's own slotof."""
    import types
    import k_ftsplit
    cpu_tier = types.SimpleNamespace(_CU=None)
    k_ftsplit.install(cpu_tier)
    pool = tier["pool"]
    rng = np.random.default_rng(70)
    bsz, H, E = 2, tier["H"], tier["E"]
    sel = torch.from_numpy(np.stack([rng.choice(E, 4, replace=False) for _ in range(bsz)]).astype(np.int64)).cuda()
    w = torch.from_numpy(rng.random((bsz, 4)).astype(np.float16)).cuda()
    z = torch.from_numpy(rng.standard_normal((bsz, H)).astype(np.float16)).cuda()
    score = torch.zeros(E, device="cuda")
    pol = torch.tensor([0.4, 0.023, 0.11, 0.104, 0.2, 32, -1, 0] + [0.0] * 12, device="cuda")
    ctrl = torch.zeros(16, dtype=torch.int64, device="cuda")
    hx = torch.zeros(bsz * H, dtype=torch.float16, device="cuda")
    hp = torch.zeros(bsz * 4 * 3, dtype=torch.int32, device="cuda")
    so, wo = torch.empty(bsz * 4, dtype=torch.int64, device="cuda"), torch.empty(bsz * 4, dtype=torch.float16, device="cuda")
    dflag, stats = torch.zeros(1, dtype=torch.int64, device="cuda"), torch.zeros(8, dtype=torch.int64, device="cuda")
    cpu_tier._CU.ft_split(sel.contiguous(), w.contiguous(), z, pool.E, pool.first, pool.slotof[0], score, pol,
                          ctrl.data_ptr(), hx.data_ptr(), hp.data_ptr(), 1, 0, 0, so, wo, dflag, stats,
                          torch.empty(0, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    # full residency: every pick is a hit, the selection passes through, nothing is published
    assert torch.equal(so.view(bsz, 4), sel) and torch.equal(wo.view(bsz, 4), w)
    assert int(dflag.item()) == 0 and stats.tolist()[:4] == [len(torch.unique(sel)), 0, 0, 1]


def test_serve_stats_after_forward(tier):
    """/stats and /ec_verify over the live tier and pool (serve_stats, glm53/serve.py:571-629)."""
    from fastapi import FastAPI
    from fastapi.testclient import TestClient
    import ft_tier
    import serve_stats
    x = torch.zeros((1, tier["H"]), dtype=torch.float32)
    sel = torch.tensor([[0, 1, 2, 3]], dtype=torch.int32)
    ft_tier.tier_forward(0, x, sel, torch.full((1, 4), 0.25), 1)
    c = TestClient(serve_stats.mount(FastAPI(), pools=[tier["pool"]]))
    r = c.get("/stats").json()
    assert r["tier"]["jobs"] >= 1 and r["tier"]["layers"] == 2
    assert r["expert_cache"] and r["expert_cache"][0]["residency"] == "full"
    v = c.get("/ec_verify").json()["verify"]
    assert all(p["bad_slots"] == 0 and p["bad_tables"] == 0 for p in v)


GPU_LI = 200   # the tier's layers li in the session context (ids no other test module registers)


@pytest.fixture
def worker(tier, gpu):
    """tier_start: the extension's device worker serves the jobs ft_split publishes to the tier's ingress buffers.
    The device share of each layer runs on a second context holding the same layers (tier_forward is refused while
    the worker runs, as in the reference)."""
    import ft_tier
    for li, L in enumerate(tier["layers"]):
        L.register(gpu, GPU_LI + li)
    tier["ctrl"].zero_()
    ft_tier.tier_start(0)
    try:
        yield tier
    finally:
        ft_tier.tier_stop()


def _split_on_tier(t, sel, w, z, slotof, pol, seq, li):
    import ft_tier
    n = sel.numel()
    so, wo = torch.empty(n, dtype=torch.int64, device="cuda"), torch.empty(n, dtype=torch.float16, device="cuda")
    dflag, stats = torch.zeros(1, dtype=torch.int64, device="cuda"), torch.zeros(8, dtype=torch.int64, device="cuda")
    ft_tier.ft_split(sel, w, z, t["E"], 0, slotof, torch.zeros(t["E"], device="cuda"), pol, t["ctrl"].data_ptr(),
                     t["hx"].data_ptr(), t["picks"].data_ptr(), seq, li, 0, so, wo, dflag, stats,
                     torch.empty(0, dtype=torch.int32, device="cuda"))
    return so, wo, dflag, stats


def test_handshake_layer_through_the_extension(worker, gpu, oracle):
    """cpu_tier's decode sequence through the extension's own entry points (ft_split, ft_combine) with the handshake
    policy (pol[7] = 1, GLM53_CT_HANDSHAKE): every layer publishes an empty job, which the worker started by
    tier_start answers on the device (hout zeroed, as run_job does), so ft_combine returns without waiting out its
    timeout (stats[6] == 0) and leaves the values of the layer output (the EXACT layer, bit for bit) as they were."""
    import ft_tier
    t = worker
    H, E = t["H"], t["E"]
    rng = np.random.default_rng(88)
    x = torch.from_numpy((rng.standard_normal((1, H)) * 0.5).astype(np.float16)).cuda()
    sel = torch.from_numpy(rng.choice(E, 4, replace=False).astype(np.int64)).cuda()
    w = torch.from_numpy(rng.random(4).astype(np.float16)).cuda()
    t["hout"].fill_(7.0)
    pol = torch.tensor([0.4, 0.023, 0.11, 0.104, 0.2, 32, -1, 1] + [0.0] * 12, device="cuda")
    pool = t["pool"]
    want = oracle.moe_forward(_experts(oracle, t["layers"][0]), x.float().cpu().numpy(),
                              sel.cpu().numpy().reshape(1, 4), w.float().cpu().numpy().reshape(1, 4), mode=1)
    for seq in (1, 2, 3):
        so, wo, dflag, stats = _split_on_tier(t, sel, w, x, pool.slotof[0], pol, seq, 0)
        out = torch.empty((1, H), dtype=torch.float32, device="cuda")
        gpu.moe_forward(GPU_LI, x, so.view(1, 4), wo.view(1, 4), out)
        torch.cuda.synchronize()
        before = out.clone()
        ft_tier.ft_combine(out, dflag, t["ctrl"].data_ptr(), t["hout"].data_ptr(), stats, 2_000_000_000)
        torch.cuda.synchronize()
        assert int(dflag.item()) == seq and int(t["ctrl"][1].item()) == seq
        assert not torch.any(t["hout"][:H])
        assert torch.equal(out, before) and np.array_equal(out.cpu().numpy(), want)
        st = stats.tolist()
        assert st[6] == 0 and st[5] == 1 and st[7] == 1


@pytest.mark.parametrize("li", [0, 1])
def test_extension_worker_computes_published_picks(worker, gpu, oracle, li):
    """A residency row with misses (experts 3..5) and the policy forcing every miss to the host lane: ft_split
    publishes those picks to the tier, the device worker computes them into hout (the reference's job order) and
    answers, ft_combine adds them to the device share: the layer is the reference's composition, bit for bit, and
    no pick is lost."""
    import ft_tier
    t = worker
    H, E, bsz = t["H"], t["E"], 3
    rng = np.random.default_rng(120 + li)
    x = torch.from_numpy((rng.standard_normal((bsz, H)) * 0.5).astype(np.float16)).cuda()
    sel = torch.from_numpy(np.stack([rng.choice(E, 4, replace=False) for _ in range(bsz)]).astype(np.int64)).cuda()
    w = torch.from_numpy((rng.random((bsz, 4)) + 0.1).astype(np.float16)).cuda()
    slotof = torch.tensor([0, 1, 2, -1, -1, -1], dtype=torch.int32, device="cuda")
    pol = torch.tensor([0.4, 0.023, 0.11, 0.104, 0.2, 32, 100, 0] + [0.0] * 12, device="cuda")
    so, wo, dflag, stats = _split_on_tier(t, sel.view(-1), w.view(-1), x, slotof, pol, 1, li)
    out = torch.empty((bsz, H), dtype=torch.float32, device="cuda")
    gpu.moe_forward(GPU_LI + li, x, so.view(bsz, 4), wo.view(bsz, 4), out)
    ft_tier.ft_combine(out, dflag, t["ctrl"].data_ptr(), t["hout"].data_ptr(), stats, 500_000_000)
    torch.cuda.synchronize()
    ctrl = t["ctrl"].cpu().numpy()
    np_ = int(ctrl[4])
    assert int(dflag.item()) == 1 and ctrl[0] == 1 and ctrl[1] == 1 and np_ > 0 and stats.tolist()[6] == 0
    picks = t["picks"].cpu().numpy()[:3 * np_].reshape(-1, 3)
    hs = np.full((bsz, 4), -1, np.int64)
    hw = np.zeros((bsz, 4), np.float32)
    cnt = [0] * bsz
    for tk, e, wb in picks:
        hs[tk, cnt[tk]] = e
        hw[tk, cnt[tk]] = np.array([wb], np.int32).view(np.float32)[0]
        cnt[tk] += 1
    ds = so.view(bsz, 4).cpu().numpy()
    for tk in range(bsz):
        assert sorted([int(e) for e in ds[tk] if e >= 0] + [int(e) for e in hs[tk] if e >= 0]) == \
            sorted(int(e) for e in sel[tk].cpu().numpy())
    ex = _experts(oracle, t["layers"][li])
    xf = x.float().cpu().numpy()
    want = (oracle.moe_forward(ex, xf, ds, wo.view(bsz, 4).float().cpu().numpy(), mode=1)
            + oracle.moe_forward(ex, xf, hs, hw, mode=1)).astype(np.float32)
    assert np.array_equal(out.cpu().numpy(), want)
    with pytest.raises(RuntimeError, match="worker running"):
        ft_tier.tier_forward(li, x.float().cpu(), sel.int().cpu(), w.float().cpu(), 1)
