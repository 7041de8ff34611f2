"""The reference-shaped Python surface (ft_tier = the tier extension, k_ftsplit.install, expert_cache.Pool) on the
CPU: names, argument checks with the reference's messages, routing-row builder against the oracle, residency
tables, hit counting and verify's corruption detection. GPU behaviour is in test_gpu_shims.py."""
import types

import numpy as np
import pytest
import torch

import fake_moe


def test_tier_surface_names():
    """The names come from the PyTorch-ROCm extension (a pybind11 module built from csrc/torch_ext.cpp), under the
    reference's pybind names (ft_tier_ext.cpp:1288-1334, ft_tier_cu.cu:296-300)."""
    import ft_tier
    import torch_ext
    ext = torch_ext.load()
    assert ext.__file__.endswith("gfl_torch_ext.so")
    for name in ("tier_init", "tier_add_layer", "tier_start", "tier_stop", "tier_forward", "tier_stats",
                 "tier_set_act_limit", "tier_set_e6", "tier_job_hist", "ft_split", "ft_combine",
                 "tier_lut_build_grouped_rows"):
        assert callable(getattr(ft_tier, name)) and getattr(ft_tier, name) is getattr(ext, name)


def test_tier_calls_before_init_fail_like_the_reference():
    import ft_tier
    assert ft_tier.tier_state()[0] is False
    with pytest.raises(RuntimeError, match="init first"):
        ft_tier.tier_add_layer(0, torch.zeros(1, 3, dtype=torch.int64), *[torch.zeros(1, 1).half()] * 6)
    with pytest.raises(RuntimeError, match="worker running"):
        ft_tier.tier_forward(0, torch.zeros(1, 256), torch.zeros(1, 8, dtype=torch.int32), torch.zeros(1, 8), 1)
    assert ft_tier.tier_stats() == []


def test_split_argument_checks():
    import ft_tier
    sel = torch.zeros(8, dtype=torch.int64)
    w = torch.zeros(8, dtype=torch.float16)
    z = torch.zeros(1, 64, dtype=torch.float16)
    args = (288, 0, torch.zeros(288, dtype=torch.int32), torch.zeros(288), torch.zeros(20), 0, 0, 0, 1, 0, 0,
            torch.empty(8, dtype=torch.int64), torch.empty(8, dtype=torch.float16), torch.zeros(1, dtype=torch.int64),
            torch.zeros(8, dtype=torch.int64), torch.empty(0, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="policy needs 20 entries"):
        ft_tier.ft_split(sel, w, z, *args[:4], torch.zeros(19), *args[5:])
    with pytest.raises(RuntimeError, match="dtypes"):
        ft_tier.ft_split(sel.int(), w, z, *args)
    with pytest.raises(RuntimeError, match="E <= 1024"):
        ft_tier.ft_split(sel, w, z, 2048, *args[1:])
    with pytest.raises(RuntimeError, match="one device"):       # CPU tensors: the split runs on the GPU
        ft_tier.ft_split(sel, w, z, *args)


def test_grouped_rows_matches_oracle_and_messages(oracle):
    import ft_tier
    rng = np.random.default_rng(21)
    T, K, E = 9, 8, 40
    sel = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int64)
    sel[2, 5] = -1
    w = rng.random((T, K)).astype(np.float16)
    w[2, 5] = 0
    take = (rng.random(E) < 0.5).astype(np.uint8)
    got = ft_tier.tier_lut_build_grouped_rows(torch.from_numpy(sel), torch.from_numpy(w), torch.from_numpy(take), E)
    want = oracle.grouped_rows(sel, w.astype(np.float32), take, E)
    for a, b in zip(got, want):
        assert np.array_equal(a.numpy(), b)
    assert [t.dtype for t in got] == [torch.int32, torch.int32, torch.int32, torch.float32]
    dup = sel.copy(); dup[0, 1] = dup[0, 0]
    with pytest.raises(RuntimeError, match="grouped duplicate expert for token"):
        ft_tier.tier_lut_build_grouped_rows(torch.from_numpy(dup), torch.from_numpy(w), torch.ones(E, dtype=torch.uint8), E)
    bad = w.copy(); bad[2, 5] = 0.5
    with pytest.raises(RuntimeError, match="grouped masked picks require zero weight"):
        ft_tier.tier_lut_build_grouped_rows(torch.from_numpy(sel), torch.from_numpy(bad), torch.from_numpy(take), E)
    with pytest.raises(RuntimeError, match="take must be contiguous CPU uint8"):
        ft_tier.tier_lut_build_grouped_rows(torch.from_numpy(sel), torch.from_numpy(w), torch.ones(E), E)


def test_k_ftsplit_install_swaps_the_handle():
    import ft_tier
    import k_ftsplit
    stock = types.SimpleNamespace(ft_split=None, ft_combine=None)
    cpu_tier = types.SimpleNamespace(_CU=stock)
    assert k_ftsplit.install(cpu_tier) is stock
    assert cpu_tier._CU.ft_combine is ft_tier.ft_combine
    n0 = k_ftsplit.STATS["fast"]
    with pytest.raises(RuntimeError, match="policy needs 20 entries"):
        z64 = torch.zeros(8, dtype=torch.int64)
        cpu_tier._CU.ft_split(z64, torch.zeros(8).half(), torch.zeros(1, 64).half(), 8, 0,
                              torch.zeros(8, dtype=torch.int32), torch.zeros(8), torch.zeros(3), 0, 0, 0, 1, 0, 0,
                              z64, torch.zeros(8).half(), z64[:1], z64, torch.empty(0, dtype=torch.int32))
    assert k_ftsplit.STATS["fast"] == n0 + 1
    t = ft_tier.install(types.SimpleNamespace())
    import torch_ext
    assert t._H is torch_ext.load() and t._CU.ft_split is ft_tier.ft_split


def _cpu_mods(L=2, E=6, H=256, I=256, seed=0):
    g = torch.Generator().manual_seed(seed)
    mods = []
    for li in range(L):
        mats = []
        for p, (k, n) in enumerate(((H, I), (H, I), (I, H))):
            mats.append([(torch.randint(0, 256, ((k // 16) * (n // 16) * 96,), generator=g, dtype=torch.uint8),
                          torch.ones(k, dtype=torch.float16), torch.ones(n, dtype=torch.float16)) for _ in range(E)])
        mods.append(fake_moe.module(f"model.layers.{li}.mlp", E, H, I, mats, "cpu"))
    return mods


def test_pool_full_residency_tables_and_steps():
    import expert_cache
    mods = _cpu_mods()
    pool = expert_cache.Pool("cpu", mods)
    L, E = 2, 6
    assert pool.E == E and pool.first == 0 and pool.S == L * E
    assert torch.equal(pool.slotof, torch.arange(L * E, dtype=torch.int32).view(L, E))
    assert (pool.slotof >= 0).all()                      # every lookup hits (cpu_tier.routed reads slotof[li])
    for li, m in enumerate(mods):
        assert m._ec == (pool, li)
        assert torch.equal(pool.home[li, :, 0], m.multi_gate.ptrs_trellis)
        assert torch.equal(pool.home[li, :, 2], m.multi_down.ptrs_trellis)
    pool.step(1, torch.tensor([[0, 5, -1, 3]]), True)
    pool.step(0, torch.tensor([2, 9]), False)              # 9 is outside this layer's local range
    s = pool.summary()
    assert s["hits"] == 4 and s["misses"] == 0 and s["residency"] == "full" and s["picks_hist"] == {2: 1, 4: 1}
    assert pool.verify() == {"device": "cpu", "bad_slots": 0, "bad_tables": 0, "owned": L * E}


def test_pool_verify_detects_corruption():
    import expert_cache
    mods = _cpu_mods(seed=1)
    pool = expert_cache.Pool("cpu", mods)
    mods[1].multi_up.linears[4].inner.trellis[17] ^= 0x40          # a flipped bit in one expert's bytes
    mods[0].multi_down.ptrs_trellis[2] += 256                       # a pointer table entry moved away from home
    r = pool.verify()
    assert r["bad_slots"] == 1 and r["bad_tables"] == 1


def test_attach_wraps_the_router_to_step_the_pool():
    import expert_cache
    mods = _cpu_mods(seed=2)
    sel = torch.tensor([[1, 2]])
    for m in mods:
        m.routing_fn = lambda bsz, cfg, z, params: (sel, torch.ones(1, 2).half())
    expert_cache.POOLS.clear()
    pools = expert_cache.attach_modules(expert_cache.find_moe(mods))
    assert len(pools) == 1
    out = mods[1].routing_fn(1, None, None, {})
    assert out[0] is sel
    mods[0].routing_fn(1, None, None, {"tp_warmup": True})        # measurement calls are not counted
    assert expert_cache.summary()[0]["hits"] == 2
    expert_cache.POOLS.clear()
