"""Serve-layer counters and the cache check for this build (glm53/serve.py:571-629 `/stats` and `/ec_verify`).

The reference's `/stats` joins the serving counters with `cpu_tier.summary()` (split hits and misses, host-tier
waits, cpu_tier.py:805-840), `expert_cache.summary()` and `k_overlap.summary()`; `/ec_verify` runs the cache's exact
consistency check. Here the same sections come from the library: the split counters (the `stats` int64 [8] tensor
ft_split and ft_combine update), the expert-call counters of the tier shim, the context's host counters and per-stage
device times, the full-residency pool and the shared-expert overlap. `mount(app)` adds both endpoints to a FastAPI
application such as the reference's serve.py.
"""
import time

# ft_split / ft_combine stats words (kernels/cpu_avx2/ft_tier_cu.cu:21-236): 0 unique hits, 1 unique misses, 2 picks
# sent to the host lane, 3 calls, 4 waited ns, 5 waits, 6 timeouts, 7 host already done when the GPU arrived
SPLIT_WORDS = ("unique_hits", "unique_misses", "cpu_experts", "calls", "wait_ns", "waits", "timeouts", "gpu_late")


def split_summary(stats):
    """The split/combine counters in cpu_tier.summary()'s terms (glm53/cpu_tier.py:805-840)."""
    st = [int(v) for v in (stats.tolist() if hasattr(stats, "tolist") else stats)][:8]
    st += [0] * (8 - len(st))
    calls = max(1, st[3])
    return {"calls": st[3], "unique_hits": st[0], "unique_misses": st[1], "cpu_experts": st[2],
            "cpu_experts_per_call": round(st[2] / calls, 3), "misses_per_call": round(st[1] / calls, 3),
            "hit_rate_unique": round(st[0] / max(1, st[0] + st[1]), 4),
            "gpu_wait_ms_per_job": round(st[4] / 1e6 / max(1, st[5]), 4), "gpu_waits": st[5], "timeouts": st[6],
            "gpu_late": st[7], "gpu_late_frac": round(st[7] / max(1, st[5]), 4)}


def context_summary(ctx):
    """Host counters of a _native.Context (gfl_stats: no device synchronisation)."""
    st = ctx.stats()
    return {"forward_calls": int(st[0]), "picks": int(st[1]), "layers": int(st[2]), "workspace_bytes": int(st[3])}


def tier_summary():
    """The tier shim's tier_stats words, named (ft_tier_ext.cpp:906-914)."""
    import ft_tier
    init, running, act_limit, nlayers = ft_tier.tier_state()
    if not init:
        return None
    h = ft_tier.tier_stats()
    return {"jobs": h[0], "experts": h[1], "tokens": h[2], "empty_jobs": h[3], "running": running,
            "act_limit": act_limit, "layers": nlayers}


def summary(split_stats=None, contexts=(), overlap=None, extra=None, pools=None):
    """The `/stats` document: {"split", "tier", "contexts", "expert_cache", "k_overlap"} plus `extra`. `pools`
    defaults to the pools expert_cache.attach created."""
    import expert_cache
    st = dict(extra or {})
    if split_stats is not None:
        st["split"] = split_summary(split_stats)
    st["tier"] = tier_summary()
    st["contexts"] = [context_summary(c) for c in contexts]
    st["expert_cache"] = expert_cache.summary() if pools is None else [p.summary() for p in pools]
    if overlap is not None:
        st["k_overlap"] = overlap.summary()
    return st


def verify(pools=None):
    """`/ec_verify`: every pool's exact consistency check and the time it took."""
    import expert_cache
    t0 = time.time()
    r = expert_cache.verify() if pools is None else [p.verify() for p in pools]
    return {"verify": r, "seconds": round(time.time() - t0, 2)}


def mount(app, split_stats=None, contexts=(), overlap=None, extra=None, pools=None):
    """Add GET /stats and GET /ec_verify to a FastAPI app. `extra` is a callable returning the server's own
    counters (the reference's G["stats"])."""
    from fastapi.responses import JSONResponse

    @app.get("/stats")
    async def stats():
        return JSONResponse(summary(split_stats, contexts, overlap, extra() if callable(extra) else extra, pools))

    @app.get("/ec_verify")
    async def ec_verify():
        return JSONResponse(verify(pools))

    return app
