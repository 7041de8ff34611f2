"""Router (gfl_route through the C ABI) against the CPU oracle's closed form (oracle.route).

Bar: bit-exact sel and w. Both sides compute e = exp(-x) correctly rounded to fp32 (the oracle in double through
libm, the device in double), s = 1 / (1 + e) and w = s / sum in fp32, fp16 rounding to nearest even. Cases cover
uniform and Zipf-skewed logits, saturated scores (many exact ties: the lower expert index wins), all-equal logits,
the widest shape (E = 1024, topk = 16), topk = E = 64, and an empty batch.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _route(logits, topk):
    import torch
    import _native
    lg = torch.from_numpy(np.ascontiguousarray(logits, dtype=np.float32)).cuda()
    sel, w = _native.route(lg, topk)
    torch.cuda.synchronize()
    return sel.cpu().numpy(), w.cpu().numpy().view(np.uint16)


def _check(oracle, logits, topk):
    got_s, got_w = _route(logits, topk)
    want_s, want_w = oracle.route(logits, topk)
    assert np.array_equal(got_s, want_s)
    assert np.array_equal(got_w, want_w)
    return got_s, got_w


@pytest.mark.parametrize("M,E,topk", [(1, 288, 8), (97, 288, 8), (33, 1024, 16), (5, 64, 64), (64, 160, 6)])
def test_route_uniform_bitexact(gpu, oracle, M, E, topk):
    rng = np.random.default_rng(M * 7 + E + topk)
    _check(oracle, rng.standard_normal((M, E)).astype(np.float32), topk)


def test_route_zipf_bitexact(gpu, oracle):
    import synth
    rng = np.random.default_rng(11)
    _check(oracle, synth.zipf_logits(128, 288, 1.1, rng), 8)


def test_route_ties_lower_index(gpu, oracle):
    rng = np.random.default_rng(12)
    logits = (rng.standard_normal((16, 288)) * 12).astype(np.float32)     # many scores saturate to exactly 1.0f
    logits[3, :] = 25.0
    logits[4, :] = 0.0
    sel, w = _check(oracle, logits, 8)
    assert list(sel[3]) == list(range(8)) and list(sel[4]) == list(range(8))
    assert np.all(w[4] == np.float16(0.125).view(np.uint16))


def test_route_empty_and_errors(gpu):
    import torch
    import _native
    lg = torch.zeros((0, 288), dtype=torch.float32, device="cuda")
    sel, w = _native.route(lg, 8)
    assert sel.shape == (0, 8)
    with pytest.raises(_native.NativeError, match="topk"):
        _native.route(torch.zeros((2, 4), dtype=torch.float32, device="cuda"), 8)


@pytest.mark.parametrize("handshake", [False, True])
def test_routing_hook_decode_layer(gpu, oracle, handshake):
    """routing.RoutingHook: routing_fn(bsz, cfg, z, params) -> the split's selection from one fused router+split
    launch, equal to the router's picks (every expert resident); the layer on that selection is the oracle's EXACT
    layer on the router's closed-form picks; the combine hook leaves its values unchanged (with the handshake policy
    the split publishes an empty job, which the hook's device worker answers, so the combine does not wait: stats[6]
    stays 0)."""
    import torch
    import _native
    import routing
    import synth
    H, I, E, li, bsz = 512, 256, 16, 63, 2
    L = synth.SynthLayer(li, E, H, I, (3, 3, 3))
    L.register(gpu, li)
    rng = np.random.default_rng(63 + handshake)
    W = torch.from_numpy((rng.standard_normal((E, H)) * 0.05).astype(np.float32)).cuda()
    z = torch.from_numpy(rng.standard_normal((bsz, H)).astype(np.float16)).cuda()
    ing = routing.Ingress(H, max_bsz=4, topk=8)
    pol = torch.tensor([0.4, 0.023, 0.11, 0.104, 0.2, 32, -1, float(handshake)] + [0.0] * 12, device="cuda")
    hook = routing.RoutingHook(W, E, 8, li, torch.arange(E, dtype=torch.int32, device="cuda"), pol, ing, ctx=gpu)
    sel, w = hook.routing_fn(bsz, None, z, {})
    out = torch.empty((bsz, H), dtype=torch.float32, device="cuda")
    gpu.moe_forward(li, z, sel, w, out)
    torch.cuda.synchronize()
    before = out.clone()
    out = hook.combine(out)
    torch.cuda.synchronize()
    logits = (z.float() @ W.t()).cpu().numpy()
    want_s, want_w = oracle.route(logits, 8)
    assert np.array_equal(sel.cpu().numpy(), want_s)
    assert np.array_equal(w.cpu().numpy().view(np.uint16), want_w)
    from oracle import Mat
    ex = []
    for e in range(E):
        ms = []
        for p in range(3):
            tr, suh, svh = L.matrix(e, p)
            k, n = (H, I) if p < 2 else (I, H)
            ms.append(Mat(tr, suh, svh, k, n, 3))
        ex.append(tuple(ms))
    want = oracle.moe_forward(ex, z.float().cpu().numpy(), want_s, want_w.view(np.float16).astype(np.float32), mode=1)
    assert torch.equal(out, before) and np.array_equal(out.cpu().numpy(), want)
    st = ing.stats.tolist()
    assert int(ing.dflag.item()) == (ing.seq if handshake else 0) and st[6] == 0
