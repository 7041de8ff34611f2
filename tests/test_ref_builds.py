"""The oracle against the reference's own engine (oracle/_ref, compiled from kernels/cpu_avx2/ft_core.h in place), in
both builds: the bitwise A/B build (-ffp-contract=off, tools/bench/kernel-ab-harness.cpp:3-5) and the server build
(glm53/cpu_tier.py:76-79 flags, GCC's default contraction).

EXACT against the A/B build is bit-exact (the oracle and the device path are pinned to it). The server build fuses
multiply-adds where the A/B build rounds twice; for EXACT that moves only last bits (reported, and held to the
north-star max-abs <= 2e-3 * RMS); AFFINE and I16 move by ~2e-3 of the RMS between the two builds.
"""
import numpy as np
import pytest


def _case(oracle, H, I, E, M, topk, seed):
    ex = [oracle.synth_expert(9, e, H, I) for e in range(E)]
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, H)).astype(np.float16).astype(np.float32)
    sel = np.stack([rng.permutation(E)[:topk] for _ in range(M)]).astype(np.int32)
    sel[rng.random(sel.shape) < 0.1] = -1
    w = rng.random(sel.shape).astype(np.float32)
    return ex, x, sel, w


def _rel(a, b):
    rms = float(np.sqrt(np.mean(b.astype(np.float64) ** 2)))
    return float(np.abs(a.astype(np.float64) - b).max()) / rms


# The reference engine keeps its scratch across calls (moe_forward's `static Fwd F`, ft_core.h:1341, grown, never
# cleared): an AFFINE call after any call at a larger H gives wrong rows (seen here: H=512 after H=1024, in either
# mode). EXACT is unaffected. So every AFFINE call to an engine runs before its first call at a larger width in this
# process: mode 0 first, at H=512, and the server-build test's AFFINE part before its config-0-width EXACT part.
@pytest.mark.parametrize("mode", [0, 1])
def test_oracle_equals_the_reference_engine(oracle, ref, mode):
    """Random layers (skipped picks, 8-token jobs and more) beyond the committed golden vectors: the oracle's EXACT and
    AFFINE layers equal the reference engine's bit for bit."""
    cases = [(512, 256, 6, 21, 4, 1), (512, 256, 6, 16, 4, 5)] + ([(1024, 512, 10, 9, 6, 2)] if mode == 1 else [])
    for (H, I, E, M, topk, seed) in cases:
        ex, x, sel, w = _case(oracle, H, I, E, M, topk, seed)
        assert np.array_equal(oracle.moe_forward(ex, x, sel, w, mode=mode), ref.moe_forward(ex, x, sel, w, mode=mode))


def test_server_build_distance(oracle, ref, ref_server):
    """EXACT of the server build against the A/B build (to which the device path is bit-exact), config-0 width."""
    # AFFINE against the oracle, which equals the A/B build (above) and keeps no state between calls
    ex, x, sel, w = _case(oracle, 512, 256, 6, 16, 4, 6)
    fa = oracle.moe_forward(ex, x, sel, w, mode=0)
    fb = ref_server.moe_forward(ex, x, sel, w, mode=0)
    print(f"AFFINE server build vs A/B build (H=512): max-abs/RMS {_rel(fb, fa):.2e}")
    assert _rel(fb, fa) <= 1e-2
    ex, x, sel, w = _case(oracle, 5120, 1536, 8, 4, 4, 3)
    a = ref.moe_forward(ex, x, sel, w, mode=1)
    b = ref_server.moe_forward(ex, x, sel, w, mode=1)
    r = _rel(b, a)
    print(f"EXACT server build vs A/B build: max-abs/RMS {r:.2e}, differing {int(np.count_nonzero(a != b))}/{a.size}")
    assert r <= 2e-3


@pytest.mark.parametrize("limit", [0.05, 0.5])
def test_swiglu_clamp_equals_the_reference_engine(oracle, ref, limit):
    """The oracle's act_mul clamp (exllamav3's semantics: u clipped to [-L, L], silu(g) capped at L; ft_core.h:123-132)
    against the reference engine's own ACT_LIMIT path, bit for bit, at limits where the clamp changes the layer."""
    ex, x, sel, w = _case(oracle, 512, 256, 6, 9, 4, 11)
    x = (x * 4).astype(np.float16).astype(np.float32)
    got = oracle.moe_forward(ex, x, sel, w, mode=1, act_limit=limit)
    assert not np.array_equal(got, oracle.moe_forward(ex, x, sel, w, mode=1))
    assert np.array_equal(got, ref.moe_forward(ex, x, sel, w, mode=1, act_limit=limit))
