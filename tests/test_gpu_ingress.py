"""The consumer side of the ingress ABI and the router wrapper, on the GPU.

* The device worker (gfl_ingress_serve, the counterpart of run_job + worker_main, ft_tier_ext.cpp:400-627,
  781-802): a job the split publishes (picks of experts the residency row marks as misses) is computed into hout and
  answered, so that the layer (device picks + combine of the host partial) is bit-exact against the oracle's
  composition of the two parts, the reference's own arithmetic (ft_combine adds the worker's fp32 partial to the
  device output, ft_tier_cu.cu:273-294). No pick is dropped and the combine never waits out its timeout.
* A job the worker cannot compute (expert or token out of range) is refused: left unanswered and reported by
  gfl_ctx_check. With no job pending, nothing is answered.
* routing.RoutingHook wraps the model's own router like cpu_tier.routed (glm53/cpu_tier.py:305-319): calls that the
  reference does not split (bsz > maxbsz, autosplit_measure, tp_warmup) get the router's picks unchanged.
* gfl_ctx_check reports relay hand-off waits that ran out of their bound (forced from the host with a zero bound, so
  every wait expires at once and each kernel still ends normally).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

H, I, E = 512, 256, 16


@pytest.fixture(scope="module")
def layer(gpu):
    import synth
    L = synth.SynthLayer(71, E, H, I, (3, 3, 3))
    L.register(gpu, 71)
    return L


def _experts(L):
    from oracle import Mat
    out = []
    for e in range(L.E):
        ms = []
        for p in range(3):
            tr, suh, svh = L.matrix(e, p)
            k, n = (L.H, L.I) if p < 2 else (L.I, L.H)
            ms.append(Mat(tr, suh, svh, k, n, L.Ks[p]))
        out.append(tuple(ms))
    return out


def _router(W):
    """A model router in routing_fn form: logits z @ W^T, then gfl_route (sigmoid top-8, fp16 weights)."""
    import _native
    calls = []

    def routing_fn(bsz, cfg, z, params):
        calls.append(bsz)
        logits = (z.reshape(bsz, -1).float() @ W.t()).contiguous()
        return _native.route(logits, 8)
    routing_fn.calls = calls
    return routing_fn


def _policy(force, handshake=0.0):
    import torch
    return torch.tensor([0.4, 0.023, 0.11, 0.104, 0.2, 32, float(force), float(handshake)] + [0.0] * 12,
                        device="cuda")


def _host_selection(picks, np_, bsz, topk=8):
    """run_job's route as a selection: token t's published picks in pick order (sel -1 / w 0 after them)."""
    sel = np.full((bsz, topk), -1, np.int64)
    w = np.zeros((bsz, topk), np.float32)
    cnt = [0] * bsz
    for t, e, wb in picks[:np_]:
        sel[t, cnt[t]] = e
        w[t, cnt[t]] = np.array([wb], np.int32).view(np.float32)[0]
        cnt[t] += 1
    return sel, w


def test_routing_hook_returns_the_routers_picks_when_it_does_not_split(gpu, layer):
    import torch
    import routing
    rng = np.random.default_rng(80)
    W = torch.from_numpy((rng.standard_normal((E, H)) * 0.05).astype(np.float32)).cuda()
    orig = _router(W)
    ing = routing.Ingress(H, max_bsz=4, topk=8)
    hook = routing.RoutingHook(E=E, topk=8, li=71, slotof=torch.arange(E, dtype=torch.int32, device="cuda"),
                               pol=_policy(-1), ingress=ing, orig=orig, ctx=gpu)
    cases = [(64, {}), (2, {"autosplit_measure": True}), (3, {"tp_warmup": True})]
    for bsz, params in cases:
        z = torch.from_numpy(rng.standard_normal((bsz, H)).astype(np.float16)).cuda()
        want_s, want_w = orig(bsz, None, z, params)
        sel, w = hook.routing_fn(bsz, None, z, params)
        torch.cuda.synchronize()
        assert torch.equal(sel, want_s) and torch.equal(w.view(torch.int16), want_w.view(torch.int16)), (bsz, params)
        assert not hook.pending and ing.seq == 0
    assert hook.bypassed == 3
    # the router-weight form bypasses the same way, through gfl_route alone
    hw = routing.RoutingHook(W, E, 8, 71, torch.arange(E, dtype=torch.int32, device="cuda"), _policy(-1), ing)
    z = torch.from_numpy(rng.standard_normal((64, H)).astype(np.float16)).cuda()
    sel, w = hw.routing_fn(64, None, z, {})
    want_s, want_w = orig(64, None, z, {})
    torch.cuda.synchronize()
    assert torch.equal(sel, want_s) and torch.equal(w.view(torch.int16), want_w.view(torch.int16))
    assert tuple(sel.shape) == (64, 8) and ing.seq == 0
    # a decode-sized call is split: at full residency the selection is the router's
    z = torch.from_numpy(rng.standard_normal((2, H)).astype(np.float16)).cuda()
    sel, w = hook.routing_fn(2, None, z, {})
    want_s, want_w = orig(2, None, z, {})
    torch.cuda.synchronize()
    assert hook.pending and ing.seq == 1 and tuple(sel.shape) == (2, 8)
    assert torch.equal(sel, want_s) and torch.equal(w.view(torch.int16), want_w.view(torch.int16))
    hook.combine(torch.zeros((2, H), dtype=torch.float32, device="cuda"))
    gpu.check()


@pytest.mark.parametrize("bsz", [1, 3, 4])
def test_device_worker_serves_published_misses_bitexact(gpu, oracle, layer, bsz):
    """slotof marks experts 8..15 as misses and the policy forces every miss to the host lane: the split publishes
    those picks, the hook's device worker computes and answers them, and the combined layer is the reference's."""
    import torch
    import routing
    rng = np.random.default_rng(81 + bsz)
    W = torch.from_numpy((rng.standard_normal((E, H)) * 0.08).astype(np.float32)).cuda()
    slotof = torch.tensor([e if e < 8 else -1 for e in range(E)], dtype=torch.int32, device="cuda")
    ing = routing.Ingress(H, max_bsz=4, topk=8, timeout_ns=500_000_000)
    hook = routing.RoutingHook(E=E, topk=8, li=71, slotof=slotof, pol=_policy(100), ingress=ing, orig=_router(W),
                               ctx=gpu)
    z = torch.from_numpy(rng.standard_normal((bsz, H)).astype(np.float16)).cuda()
    router_sel, router_w = hook.orig(bsz, None, z, {})
    sel, w = hook.routing_fn(bsz, None, z, {})
    out = torch.empty((bsz, H), dtype=torch.float32, device="cuda")
    gpu.moe_forward(71, z, sel.contiguous(), w.contiguous(), out)
    out = hook.combine(out)
    torch.cuda.synchronize()
    gpu.check()
    ctrl = ing.ctrl.cpu().numpy()
    np_ = int(ctrl[4])
    assert ctrl[0] == ing.seq == 1 and ctrl[1] == ctrl[0] and ctrl[3] == bsz and np_ > 0
    st = ing.stats.cpu().numpy()
    assert st[6] == 0 and st[5] == 1
    picks = ing.picks.cpu().numpy()[:3 * np_].reshape(-1, 3)
    # every router pick is computed exactly once: on the device or by the worker
    rs, rw = router_sel.cpu().numpy(), router_w.cpu().numpy()
    ds = sel.cpu().numpy()
    for t in range(bsz):
        dev = sorted(int(e) for e in ds[t] if e >= 0)
        host = sorted(int(e) for tt, e, _ in picks if tt == t)
        assert sorted(dev + host) == sorted(int(e) for e in rs[t]) and all(e >= 8 for e in host), t
    x = z.float().cpu().numpy()
    ex = _experts(layer)
    want_dev = oracle.moe_forward(ex, x, ds, w.cpu().numpy().astype(np.float32), mode=1)
    hs, hw = _host_selection(picks, np_, bsz)
    want_host = oracle.moe_forward(ex, x, hs, hw, mode=1)
    assert np.array_equal(ing.hout[:bsz * H].cpu().numpy().reshape(bsz, H), want_host)
    want = (want_dev + want_host).astype(np.float32)
    assert np.array_equal(out.cpu().numpy(), want)


def test_device_worker_refuses_and_answers(gpu, oracle, layer):
    """Hand-made jobs: one naming an expert outside the layer is refused (left unanswered, reported by
    gfl_ctx_check); a valid one is computed in run_job's order and answered; with nothing pending nothing is."""
    import torch
    import _native
    bsz = 2
    rng = np.random.default_rng(90)
    hx = torch.from_numpy(rng.standard_normal((bsz, H)).astype(np.float16)).cuda()
    hout = torch.full((bsz * H,), 3.0, dtype=torch.float32, device="cuda")
    ctrl = torch.zeros(16, dtype=torch.int64, device="cuda")

    def job(seq, done, picks, ntok=bsz, li=71):
        ctrl.copy_(torch.tensor([seq, done, li, ntok, len(picks)] + [0] * 11, dtype=torch.int64))
        arr = np.zeros((max(1, len(picks)), 3), np.int32)
        for i, (t, e, wv) in enumerate(picks):
            arr[i] = (t, e, np.array([wv], np.float32).view(np.int32)[0])
        return torch.from_numpy(arr.reshape(-1)).cuda()

    hp = job(5, 4, [(0, 3, 0.5), (1, E + 3, 0.25)])
    gpu.ingress_serve(71, bsz, 8, ctrl.data_ptr(), hx.data_ptr(), hp.data_ptr(), hout.data_ptr())
    torch.cuda.synchronize()
    assert int(ctrl[1].item()) == 4
    with pytest.raises(_native.NativeError, match="refused"):
        gpu.check()
    gpu.check()                                   # the status words were cleared
    hp = job(6, 5, [(0, 3, 0.5)], li=70)          # another layer's job
    gpu.ingress_serve(71, bsz, 8, ctrl.data_ptr(), hx.data_ptr(), hp.data_ptr(), hout.data_ptr())
    with pytest.raises(_native.NativeError, match="refused"):
        gpu.check()
    picks = [(0, 2, 0.5), (1, 5, 0.25), (0, 7, 0.125), (1, 2, 1.0)]
    hp = job(7, 6, picks)
    gpu.ingress_serve(71, bsz, 8, ctrl.data_ptr(), hx.data_ptr(), hp.data_ptr(), hout.data_ptr())
    torch.cuda.synchronize()
    gpu.check()
    assert int(ctrl[1].item()) == 7
    bits = [(t, e, int(np.array([wv], np.float32).view(np.int32)[0])) for t, e, wv in picks]
    hs, hw = _host_selection(bits, len(bits), bsz)
    assert list(hs[0][:2]) == [2, 7] and list(hs[1][:2]) == [5, 2]
    want = oracle.moe_forward(_experts(layer), hx.float().cpu().numpy(), hs, hw, mode=1)
    assert np.array_equal(hout.cpu().numpy().reshape(bsz, H), want)
    # nothing pending (ctrl[0] == ctrl[1]): hout zeroed, the done word untouched
    gpu.ingress_serve(71, bsz, 8, ctrl.data_ptr(), hx.data_ptr(), hp.data_ptr(), hout.data_ptr())
    torch.cuda.synchronize()
    gpu.check()
    assert int(ctrl[1].item()) == 7 and not torch.any(hout)


def test_ctx_check_reports_expired_relay_waits(gpu, layer, monkeypatch):
    """A zero bound on the relay hand-off wait (GFL_RELAY_SPIN_LIMIT=0, set before the context is made) makes every
    wait expire at once; the kernels finish normally and gfl_ctx_check reports the expiries, then clears them. The
    default bound reports nothing on the same call."""
    import torch
    import _native
    monkeypatch.setenv("GFL_RELAY_SPIN_LIMIT", "0")
    ctx = _native.Context(0)
    monkeypatch.delenv("GFL_RELAY_SPIN_LIMIT")
    layer.register(ctx, 71)
    rng = np.random.default_rng(95)
    x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float16)).cuda()
    sel = torch.from_numpy(rng.permutation(E)[:8].reshape(1, 8).astype(np.int64)).cuda()
    w = torch.full((1, 8), 0.125, dtype=torch.float16, device="cuda")
    out = torch.empty((1, H), dtype=torch.float32, device="cuda")
    ctx.moe_forward(71, x, sel, w, out)           # 8 picks at I = 256: the relay launches, 4 waves per column
    with pytest.raises(_native.NativeError, match="expired"):
        ctx.check()
    ctx.check()
    ctx.close()
    gpu.moe_forward(71, x, sel, w, out)
    gpu.check()
