"""ft_split / ft_combine on the GPU (gfl_split, gfl_combine through the C ABI) against the CPU oracle.

Bar: bit-exact. Every output the reference's split writes is compared: sel_out, w_out, dflag, stats[0..3], and for a
published host job the control words ctrl[0], ctrl[2..4], the pick list hpicks (token, local expert, fp32 weight bits)
and the x rows hx. The device and the oracle evaluate the cost model with the same uncontracted float expressions,
so they agree at near-ties too. Cases sweep residency (all hit, mixed, all miss), the policy vector (forced count,
per-call cap, publish flag, LUT cost table, the resident-tier lane with rres), layer-local id offsets with ids of
other layers, -1 sentinels, zero and NaN weights, keep_ids, and the size limits (1024 picks, 1024 experts).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _pol(rng, kind):
    p = np.zeros(20, np.float32)
    p[:5] = [rng.uniform(0.1, 0.6), rng.uniform(0.01, 0.05), rng.uniform(0.05, 0.3), rng.uniform(0.05, 0.2),
             rng.uniform(0.0, 0.4)]
    p[5] = rng.choice([0, 3, 32])
    p[6] = -1 if kind != "force" else rng.choice([0, 2, 100])
    p[7] = float(rng.random() < 0.3)
    if kind == "lut":
        p[11:20] = np.sort(rng.uniform(0.05, 0.6, 9)).astype(np.float32)
        p[12] = max(p[12], 0.01)
    if kind == "tri":
        p[8], p[9], p[10] = 1.0, rng.uniform(0.02, 0.2), rng.uniform(0.02, 0.2)
    return p


def _case(rng, E, first, bsz, topk, hit_rate, kind):
    H = 64
    lo, hi = first - 3, first + E + 3
    sel = np.stack([rng.choice(np.arange(lo, hi), topk, replace=False) for _ in range(bsz)]).astype(np.int64)
    w = rng.uniform(0.01, 1.0, sel.shape).astype(np.float16)
    drop = rng.random(sel.shape) < 0.08
    sel[drop] = -1
    w[drop] = 0
    w[rng.random(sel.shape) < 0.05] = 0
    wb = w.view(np.uint16).copy()
    if rng.random() < 0.2:
        wb.reshape(-1)[rng.integers(wb.size)] = 0x7E00          # a NaN weight counts as a nonzero pick
    z = rng.standard_normal((bsz, H)).astype(np.float16).view(np.uint16)
    slotof = np.where(rng.random(E) < hit_rate, rng.integers(0, 4096, E), -1).astype(np.int32)
    score = (np.round(rng.random(E) * 8) / 8).astype(np.float32)      # ties exercise the id tie-break
    rres = (rng.random(E) < 0.5).astype(np.int32) if kind == "tri" else None
    return dict(sel=sel, w=wb, z=z, E=E, first=first, slotof=slotof, score=score, pol=_pol(rng, kind),
                seq=int(rng.integers(1, 1 << 40)), li=int(rng.integers(0, 42)), keep_ids=int(rng.integers(0, 2)),
                rres=rres, stats0=rng.integers(0, 1000, 8).astype(np.int64))


def _run_gpu(c):
    import torch
    import _native
    dev = "cuda"
    sel = torch.from_numpy(c["sel"].reshape(-1).copy()).to(dev)
    w = torch.from_numpy(c["w"].reshape(-1).view(np.int16).copy()).to(dev)
    z = torch.from_numpy(c["z"].view(np.int16).copy()).to(dev)
    bsz, H = c["z"].shape
    n = sel.numel()
    ctrl = torch.zeros(16, dtype=torch.int64, device=dev)
    hx = torch.zeros(bsz * H, dtype=torch.int16, device=dev)
    hpicks = torch.full((n * 3,), -7, dtype=torch.int32, device=dev)
    sel_out = torch.empty(n, dtype=torch.int64, device=dev)
    w_out = torch.empty(n, dtype=torch.int16, device=dev)
    dflag = torch.full((1,), -5, dtype=torch.int64, device=dev)
    stats = torch.from_numpy(c["stats0"].copy()).to(dev)
    rres = torch.from_numpy(c["rres"]).to(dev) if c["rres"] is not None else torch.empty(0, dtype=torch.int32,
                                                                                          device=dev)
    _native.split(sel, w, z.view(bsz, H), c["E"], c["first"], torch.from_numpy(c["slotof"]).to(dev),
                  torch.from_numpy(c["score"]).to(dev), torch.from_numpy(c["pol"]).to(dev), ctrl.data_ptr(),
                  hx.data_ptr(), hpicks.data_ptr(), c["seq"], c["li"], c["keep_ids"], sel_out, w_out, dflag, stats,
                  rres)
    torch.cuda.synchronize()
    return dict(sel_out=sel_out.cpu().numpy(), w_out=w_out.cpu().numpy().view(np.uint16),
                dflag=int(dflag.item()), stats=stats.cpu().numpy(), ctrl=ctrl.cpu().numpy(),
                hx=hx.cpu().numpy().view(np.uint16), hpicks=hpicks.cpu().numpy())


def _check(oracle, c, tag):
    g = _run_gpu(c)
    r = oracle.split(c["sel"], c["w"], c["z"], c["E"], c["first"], c["slotof"], c["score"], c["pol"], c["seq"],
                     c["li"], c["keep_ids"], rres=c["rres"], stats=c["stats0"].copy())
    assert np.array_equal(g["sel_out"], r["sel_out"]), tag
    assert np.array_equal(g["w_out"], r["w_out"]), tag
    assert g["dflag"] == r["dflag"], tag
    assert np.array_equal(g["stats"][:4], r["stats"][:4]), tag
    assert np.array_equal(g["stats"][4:], c["stats0"][4:]), tag
    if r["dflag"]:
        npk = int(r["ctrl"][4])
        assert g["ctrl"][0] == r["ctrl"][0] == c["seq"], tag
        assert np.array_equal(g["ctrl"][2:5], r["ctrl"][2:5]), tag
        assert np.array_equal(g["hpicks"][:3 * npk].reshape(-1, 3), r["hpicks"]), tag
        assert np.array_equal(g["hx"], c["z"].reshape(-1)), tag
        # the split never answers a job itself (its consumer, a host or the device worker, writes ctrl[1])
        assert g["ctrl"][1] == 0, tag
    else:
        assert not g["ctrl"].any(), tag
        assert (g["hpicks"] == -7).all(), tag
    return bool(r["dflag"])


@pytest.mark.parametrize("kind", ["stock", "force", "lut", "tri"])
def test_split_matches_oracle(gpu, oracle, kind):
    rng = np.random.default_rng({"stock": 31, "force": 32, "lut": 33, "tri": 34}[kind])
    published = 0
    for i in range(60):
        E = int(rng.choice([8, 64, 288]))
        first = int(rng.choice([0, 5, 288]))
        bsz = int(rng.choice([1, 2, 3, 4, 8]))
        hit = float(rng.choice([1.0, 0.7, 0.3, 0.0]))
        c = _case(rng, E, first, bsz, 8, hit, kind)
        published += _check(oracle, c, f"{kind} case {i}: E={E} first={first} bsz={bsz} hit={hit}")
    assert published > 10


def test_split_all_resident_identity_and_stats(gpu, oracle):
    rng = np.random.default_rng(35)
    c = _case(rng, 288, 0, 4, 8, 1.0, "stock")
    c["pol"][7] = 0
    assert not _check(oracle, c, "all resident")
    g = _run_gpu(c)
    assert np.array_equal(g["sel_out"], c["sel"].reshape(-1))
    assert np.array_equal(g["w_out"], c["w"].reshape(-1))


def test_split_size_limits(gpu, oracle):
    rng = np.random.default_rng(36)
    for hit in (1.0, 0.5, 0.0):
        c = _case(rng, 1024, 0, 128, 8, hit, "stock")         # n = 1024 picks, E = 1024
        _check(oracle, c, f"limits hit={hit}")
        c = _case(rng, 1024, 0, 64, 16, hit, "lut")          # topk 16
        _check(oracle, c, f"limits topk16 hit={hit}")


def _combine_gpu(out_np, dflag, ctrl_np, hout_np, stats_np, timeout_ns):
    import torch
    import _native
    is_half = out_np.dtype == np.uint16
    out = torch.from_numpy(out_np.view(np.int16) if is_half else out_np.copy()).cuda()
    if is_half:
        out = out.view(torch.float16)
    dfl = torch.tensor([dflag], dtype=torch.int64, device="cuda")
    ctrl = torch.from_numpy(ctrl_np.copy()).cuda()
    hout = torch.from_numpy(hout_np.copy()).cuda()
    stats = torch.from_numpy(stats_np.copy()).cuda()
    _native.combine(out, dfl, ctrl.data_ptr(), hout.data_ptr(), stats, timeout_ns)
    torch.cuda.synchronize()
    o = out.view(torch.int16).cpu().numpy().view(np.uint16) if is_half else out.cpu().numpy()
    return o, stats.cpu().numpy()


@pytest.mark.parametrize("half", [False, True])
def test_combine_matches_oracle(gpu, oracle, half):
    rng = np.random.default_rng(37 + half)
    for n in (1, 5120, 4 * 5120, 128 * 5120 + 3):
        base = rng.standard_normal(n).astype(np.float32)
        out0 = base.astype(np.float16).view(np.uint16) if half else base
        hout = rng.standard_normal(n).astype(np.float32)
        seq = int(rng.integers(1, 1 << 40))
        ctrl = np.zeros(16, np.int64); ctrl[1] = seq; ctrl[4] = 3     # a job with picks
        stats0 = np.zeros(8, np.int64)
        got, st = _combine_gpu(out0.copy(), seq, ctrl, hout, stats0, 2_000_000_000)
        want = out0.copy()
        assert oracle.combine(want, seq, ctrl, hout) == 1
        assert np.array_equal(got, want), f"n={n}"
        assert list(st[5:8]) == [1, 0, 1]        # one wait, no timeout, host already done
        # no job published: output untouched, no counters
        got, st = _combine_gpu(out0.copy(), 0, ctrl, hout, stats0, 2_000_000_000)
        assert np.array_equal(got, out0) and not st.any()


def test_combine_timeout_drops_partial(gpu):
    """A done word behind the job's sequence: bounded wait, then the partial is dropped and the timeout counted."""
    rng = np.random.default_rng(39)
    n = 4 * 5120
    out0 = rng.standard_normal(n).astype(np.float32)
    ctrl = np.zeros(16, np.int64); ctrl[1] = 41
    got, st = _combine_gpu(out0.copy(), 42, ctrl, np.ones(n, np.float32), np.zeros(8, np.int64), 20_000)
    assert np.array_equal(got, out0)
    assert st[5] == 1 and st[6] == 1 and st[7] == 0
    assert 15_000 <= st[4] <= 50_000_000     # waited about the timeout (wall-clock ticks converted to ns)


def test_combine_adds_hout_of_an_empty_job(gpu):
    """A job without picks (ctrl[4] == 0) is combined like any other: out += hout, which its worker zeroed (run_job,
    ft_tier_ext.cpp:431-435), so -0 + 0 = +0; the combine itself does not look at ctrl[4] (ft_tier_cu.cu:205-235)."""
    n = 5120
    out0 = np.random.default_rng(40).standard_normal(n).astype(np.float32)
    out0[:3] = [-0.0, 0.0, -1.5]
    ctrl = np.zeros(16, np.int64); ctrl[0] = ctrl[1] = 9
    got, st = _combine_gpu(out0.copy(), 9, ctrl, np.zeros(n, np.float32), np.zeros(8, np.int64), 10**9)
    assert np.array_equal(got, out0 + np.float32(0.0)) and np.signbit(got[0]) == False
    assert list(st[5:8]) == [1, 0, 1]
    hout = np.full(n, 123.0, np.float32)
    got, st = _combine_gpu(out0.copy(), 9, ctrl, hout, np.zeros(8, np.int64), 10**9)
    assert np.array_equal(got, (out0 + hout).astype(np.float32))


def _route_split_gpu(logits, topk, c):
    import torch
    import _native
    dev = "cuda"
    M = logits.shape[0]
    lg = torch.from_numpy(logits).to(dev)
    z = torch.from_numpy(c["z"].view(np.int16).copy()).to(dev)
    H = c["z"].shape[1]
    n = M * topk
    sel = torch.empty((M, topk), dtype=torch.int64, device=dev)
    w = torch.empty((M, topk), dtype=torch.int16, device=dev)
    ctrl = torch.zeros(16, dtype=torch.int64, device=dev)
    hx = torch.zeros(M * H, dtype=torch.int16, device=dev)
    hpicks = torch.full((n * 3,), -7, dtype=torch.int32, device=dev)
    sel_out = torch.empty(n, dtype=torch.int64, device=dev)
    w_out = torch.empty(n, dtype=torch.int16, device=dev)
    dflag = torch.zeros(1, dtype=torch.int64, device=dev)
    stats = torch.zeros(8, dtype=torch.int64, device=dev)
    rres = torch.from_numpy(c["rres"]).to(dev) if c["rres"] is not None else None
    _native.route_split(lg, topk, z, c["E"], c["first"], torch.from_numpy(c["slotof"]).to(dev),
                        torch.from_numpy(c["score"]).to(dev), torch.from_numpy(c["pol"]).to(dev), ctrl.data_ptr(),
                        hx.data_ptr(), hpicks.data_ptr(), c["seq"], c["li"], c["keep_ids"], sel, w, sel_out, w_out,
                        dflag, stats, rres)
    torch.cuda.synchronize()
    return dict(sel=sel.cpu().numpy(), w=w.cpu().numpy().view(np.uint16), sel_out=sel_out.cpu().numpy(),
                w_out=w_out.cpu().numpy().view(np.uint16), dflag=int(dflag.item()), stats=stats.cpu().numpy(),
                ctrl=ctrl.cpu().numpy(), hpicks=hpicks.cpu().numpy(), hx=hx.cpu().numpy().view(np.uint16))


@pytest.mark.parametrize("kind", ["stock", "tri", "lut"])
def test_route_split_matches_router_then_split(gpu, oracle, kind):
    """gfl_route_split = the router (closed form, checked against the oracle's) followed by the split (the oracle's),
    on every output: one launch up to 4 tokens, the router's grid then the split above (5 to 128 tokens)."""
    rng = np.random.default_rng({"stock": 51, "tri": 52, "lut": 53}[kind])
    for i in range(21):
        M = [1, 2, 4, 5, 16, 64, 128][i % 7]
        E = int(rng.choice([64, 288]))
        logits = rng.standard_normal((M, E)).astype(np.float32)
        c = _case(rng, E, 0, M, 8, float(rng.choice([1.0, 0.5, 0.0])), kind)
        g = _route_split_gpu(logits, 8, c)
        sel, w = oracle.route(logits, 8)
        assert np.array_equal(g["sel"], sel) and np.array_equal(g["w"], w.reshape(g["w"].shape)), i
        r = oracle.split(sel, w, c["z"], E, 0, c["slotof"], c["score"], c["pol"], c["seq"], c["li"], c["keep_ids"],
                         rres=c["rres"])
        assert np.array_equal(g["sel_out"], r["sel_out"]) and np.array_equal(g["w_out"], r["w_out"]), i
        assert g["dflag"] == r["dflag"] and np.array_equal(g["stats"][:4], r["stats"][:4]), i
        if r["dflag"]:
            npk = int(r["ctrl"][4])
            assert np.array_equal(g["ctrl"][2:5], r["ctrl"][2:5]) and g["ctrl"][0] == c["seq"], i
            assert np.array_equal(g["hpicks"][:3 * npk].reshape(-1, 3), r["hpicks"]), i


def test_handshake_layer_does_not_wait(gpu):
    """cpu_tier's decode sequence at full residency with the handshake policy (pol[7] = 1, GLM53_CT_HANDSHAKE):
    ft_split publishes an empty job every layer and leaves it unanswered (the reference's handshake); the device
    worker (gfl_ingress_serve) answers it as the reference's worker does, zeroing hout; the layer runs on the device
    and ft_combine returns without waiting out its timeout (stats[6] == 0) and leaves the layer output's values as
    they were."""
    import torch
    import _native
    import synth
    H, I, E = 512, 256, 16
    L = synth.SynthLayer(60, E, H, I, (3, 3, 3))
    L.register(gpu, 60)
    rng = np.random.default_rng(61)
    x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float16)).cuda()
    (sel, w16), _ = synth.route_uniform(1, E, 8, rng)
    sel_d = torch.from_numpy(sel).cuda()
    w_d = torch.from_numpy(w16.view(np.int16)).cuda().view(torch.float16)
    ctrl = torch.zeros(16, dtype=torch.int64, device="cuda")
    hx = torch.zeros(H, dtype=torch.float16, device="cuda")
    hp = torch.zeros(8 * 3, dtype=torch.int32, device="cuda")
    hout = torch.full((H,), 7.0, dtype=torch.float32, device="cuda")
    so, wo = torch.empty(8, dtype=torch.int64, device="cuda"), torch.empty(8, dtype=torch.float16, device="cuda")
    dflag, stats = torch.zeros(1, dtype=torch.int64, device="cuda"), torch.zeros(8, dtype=torch.int64, device="cuda")
    pol = torch.tensor([0.4, 0.023, 0.11, 0.104, 0.2, 32, -1, 1] + [0.0] * 12, device="cuda")
    out = torch.empty((1, H), dtype=torch.float32, device="cuda")
    for seq in (1, 2, 3):
        _native.split(sel_d.view(-1), w_d.view(-1), x, E, 0, torch.arange(E, dtype=torch.int32, device="cuda"),
                      torch.zeros(E, device="cuda"), pol, ctrl.data_ptr(), hx.data_ptr(), hp.data_ptr(), seq, 60, 0,
                      so, wo, dflag, stats, None)
        torch.cuda.synchronize()
        assert int(ctrl[0].item()) == seq and int(ctrl[1].item()) == seq - 1   # published, not answered by the split
        gpu.ingress_serve(60, 1, 8, ctrl.data_ptr(), hx.data_ptr(), hp.data_ptr(), hout.data_ptr())
        gpu.moe_forward(60, x, so.view(1, 8), wo.view(1, 8), out)
        torch.cuda.synchronize()
        assert not torch.any(hout)
        before = out.clone()
        _native.combine(out, dflag, ctrl.data_ptr(), hout.data_ptr(), stats, 2_000_000_000)
        torch.cuda.synchronize()
        assert int(dflag.item()) == seq and int(ctrl[0].item()) == seq and int(ctrl[1].item()) == seq
        assert torch.equal(out, before)
    st = stats.tolist()
    assert st[6] == 0 and st[5] == 3 and st[7] == 3 and st[3] == 3
