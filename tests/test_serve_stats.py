"""Serve-layer counters (serve_stats, the counterpart of glm53/serve.py:571-629) on the CPU: the split counters in
cpu_tier.summary()'s terms, and the /stats and /ec_verify endpoints mounted on a FastAPI app."""
import numpy as np


def test_split_summary_terms():
    import serve_stats
    st = np.array([30, 10, 4, 8, 2_000_000, 4, 1, 2], np.int64)
    s = serve_stats.split_summary(st)
    assert s["calls"] == 8 and s["unique_hits"] == 30 and s["unique_misses"] == 10 and s["cpu_experts"] == 4
    assert s["hit_rate_unique"] == 0.75 and s["misses_per_call"] == 1.25 and s["cpu_experts_per_call"] == 0.5
    assert s["gpu_wait_ms_per_job"] == 0.5 and s["timeouts"] == 1 and s["gpu_late_frac"] == 0.5
    assert serve_stats.split_summary([0] * 8)["hit_rate_unique"] == 0.0


def test_endpoints_on_fastapi():
    from fastapi import FastAPI
    from fastapi.testclient import TestClient
    import serve_stats
    app = serve_stats.mount(FastAPI(), split_stats=np.array([5, 1, 0, 2, 0, 0, 0, 0], np.int64),
                            extra=lambda: {"requests": 3})
    c = TestClient(app)
    r = c.get("/stats").json()
    assert r["requests"] == 3 and r["split"]["calls"] == 2 and r["split"]["unique_hits"] == 5
    assert r["contexts"] == [] and isinstance(r["expert_cache"], list)
    v = c.get("/ec_verify").json()
    assert "verify" in v and v["seconds"] >= 0
