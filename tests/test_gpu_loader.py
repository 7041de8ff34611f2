"""EXL3 checkpoint -> HBM arenas -> registered layers (exl3_loader.load) on the GPU: layers served straight from the
loaded arenas are bit-exact against the oracle run on the same tensors read back from the files; the shared expert
lands in a k_overlap.SharedOverlap; the reference's tier self-test formula (cpu_tier.py:738-770) stays within the
expected accumulation error."""
import numpy as np
import pytest

import ckpt_synth

pytestmark = pytest.mark.gpu

H, I, E = 512, 256, 5
KS = {2: (3, 3, 3), 4: (4, 4, 3)}


@pytest.fixture(scope="module")
def loaded(gpu, tmp_path_factory):
    import exl3_loader
    import k_overlap
    tmp = tmp_path_factory.mktemp("ckpt")
    paths = ckpt_synth.write(tmp, [2, 4], E=E, H=H, I=I, Ks_by_layer=KS)
    so = k_overlap.SharedOverlap(0)
    res = exl3_loader.load(paths, gpu, shared=so)
    return dict(paths=paths, res=res, so=so)


@pytest.mark.parametrize("L", [2, 4])
def test_loaded_layer_bitexact(gpu, oracle, loaded, L):
    import torch
    rng = np.random.default_rng(L)
    M = 3
    x16 = (rng.standard_normal((M, H)) * 0.5).astype(np.float16)
    sel = np.stack([rng.permutation(E)[:3] for _ in range(M)]).astype(np.int64)
    w = rng.random(sel.shape).astype(np.float32)
    xd = torch.from_numpy(x16.view(np.int16)).view(torch.float16).cuda()
    out = torch.empty((M, H), dtype=torch.float32, device="cuda")
    gpu.moe_forward(L, xd, torch.from_numpy(sel).cuda(), torch.from_numpy(w).cuda(), out)
    torch.cuda.synchronize()
    ex = ckpt_synth.host_experts(loaded["paths"], L, E, H, I, KS[L])
    want = oracle.moe_forward(ex, x16.astype(np.float32), sel, w, mode=1)
    assert np.array_equal(out.cpu().numpy(), want)
    # the shared expert, through the side-stream path
    sh = ckpt_synth.host_experts(loaded["paths"], L, E, H, I, KS[L], shared=True)[0]
    both = torch.empty_like(out)
    loaded["so"].forward(gpu, L, xd, torch.from_numpy(sel).cuda(), torch.from_numpy(w).cuda(), both)
    torch.cuda.synchronize()
    shared = oracle.expert_forward(sh, x16.astype(np.float32), mode=1)
    assert np.array_equal(both.cpu().numpy(), (want + shared).astype(np.float32))


def test_self_test_formula(gpu, loaded):
    import exl3_loader
    r = exl3_loader.self_test(gpu, loaded["res"][2], 2)
    assert r["EXACT"] < 3e-3, r
