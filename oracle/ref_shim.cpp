// C entry points over the reference's own AVX2 expert engine (kernels/cpu_avx2/ft_core.h), compiled from the
// reference tree where it lies (oracle/Makefile, -I<reference>/kernels/cpu_avx2). TEST INFRASTRUCTURE ONLY: it
// pins the oracle (golden vectors) and is the timed CPU baseline (`cpu_baseline.kind = "reference"` in bench.py).
// Nothing in the product library links it. The reference engine is K=3 only (ft_core.h:30-31).
#include "ft_core.h"
#include <sched.h>

namespace {
Pool* g_pool = nullptr;   // heap-held: worker threads are never joined by a static destructor at exit
int g_threads = 0;

Mat mk(const uint8_t* tr, const uint16_t* suh, const uint16_t* svh, int k, int n) { Mat m; m.tr = tr; m.suh = suh; m.svh = svh; m.k = k; m.n = n; m.swz = 0; return m; }

void build_layer(Layer& L, int E, int H, int I, const uint8_t* const* tr, const uint16_t* const* sc)
{
    // tr: [E*3] gate/up/down trellis; sc: [E*6] suh_g, svh_g, suh_u, svh_u, suh_d, svh_d
    L.H = H; L.I = I; L.ex.resize(E);
    for (int e = 0; e < E; ++e)
    {
        L.ex[e].g = mk(tr[e * 3 + 0], sc[e * 6 + 0], sc[e * 6 + 1], H, I);
        L.ex[e].u = mk(tr[e * 3 + 1], sc[e * 6 + 2], sc[e * 6 + 3], H, I);
        L.ex[e].d = mk(tr[e * 3 + 2], sc[e * 6 + 4], sc[e * 6 + 5], I, H);
    }
}
}  // namespace

extern "C" {

// init_perm + init_tables, and a pool of `threads` workers pinned to `cpus` (the calling thread's affinity is restored,
// as tier_init does, ft_tier_ext.cpp:145-147)
int ref_init(int threads, const int* cpus, int ncpus)
{
    init_perm();
    init_tables();
    if (g_pool) return g_threads;
    std::vector<int> c(cpus, cpus + ncpus);
    if (c.empty()) c.push_back(0);
    cpu_set_t saved;
    sched_getaffinity(0, sizeof(saved), &saved);
    g_pool = new Pool();
    g_pool->start(threads, c);
    sched_setaffinity(0, sizeof(saved), &saved);
    g_threads = threads;
    return threads;
}

void ref_shutdown()
{
    if (g_pool) { g_pool->stop(); g_pool = nullptr; }
}

// dense_weights (ft_core.h:1657): fp32 W[k][n] holding fp16 values
void ref_dense_weights(const uint8_t* tr, int k, int n, float* W)
{
    init_perm();
    const std::vector<float> v = dense_weights(mk(tr, nullptr, nullptr, k, n));
    std::memcpy(W, v.data(), v.size() * 4);
}

uint16_t ref_state(const uint16_t* packed, int t) { return state_scalar(packed, t); }
float ref_w_gpu(uint16_t st) { return w_gpu(st); }

void ref_prep_block(const float* x, const uint16_t* suh, float* xt) { prep_block(x, suh, xt); }
void ref_out_block(float* y, const uint16_t* svh) { out_block(y, svh); }

// moe_forward (ft_core.h:1338): x fp32 [ntok][H]; sel int32 [ntok][topk] (<0 skipped); w fp32; out fp32 [ntok][H]
int ref_moe_forward(int E, int H, int I, const uint8_t* const* tr, const uint16_t* const* sc, const float* x, int ntok,
                    const int32_t* sel, const float* w, int topk, float* out, int mode, float act_limit)
{
    if (!g_pool) return -1;
    init_perm();
    init_tables();
    ACT_LIMIT = act_limit;
    Layer L;
    build_layer(L, E, H, I, tr, sc);
    std::vector<std::vector<std::pair<int, float>>> route(ntok);
    for (int t = 0; t < ntok; ++t)
        for (int j = 0; j < topk; ++j)
            if (sel[t * topk + j] >= 0) route[t].push_back({ sel[t * topk + j], w[t * topk + j] });
    moe_forward(*g_pool, L, x, ntok, route, out, mode);
    ACT_LIMIT = 0.0f;
    return 0;
}

// ref_expert (ft_core.h:1684): fp64-accumulated single expert, one token
void ref_expert64(int H, int I, const uint8_t* const* tr, const uint16_t* const* sc, const float* x, float* y)
{
    init_perm();
    Layer L;
    build_layer(L, 1, H, I, tr, sc);
    std::vector<float> W[3] = { dense_weights(L.ex[0].g), dense_weights(L.ex[0].u), dense_weights(L.ex[0].d) };
    ref_expert(L.ex[0], W, x, y);
}

// Decode-call timing in the style of tools/bench/kernel-ab-harness.cpp HARNESS_TIME (:51-105): `iters` calls of
// `ntok` tokens x `topk` experts each, expert sets cycling through the E-expert pool so weights come from DRAM, after
// `warmup` untimed calls. x fp32 [ntok][H]. Writes per-call wall seconds into `secs` (length iters). Token t of call
// `it` picks experts (it*ntok*topk + t*topk + q) % E, q < topk: distinct experts within and across the call's tokens
// while ntok*topk <= E (the union is ntok*topk experts, the uniform-routing worst case).
int ref_time_decode(int E, int H, int I, const uint8_t* const* tr, const uint16_t* const* sc, const float* x,
                    int ntok, int topk, int iters, int warmup, int mode, double* secs)
{
    if (!g_pool) return -1;
    init_perm();
    init_tables();
    Layer L;
    build_layer(L, E, H, I, tr, sc);
    std::vector<float> out((size_t)ntok * H);
    for (int it = 0; it < warmup + iters; ++it)
    {
        std::vector<std::vector<std::pair<int, float>>> route(ntok);
        for (int t = 0; t < ntok; ++t)
            for (int q = 0; q < topk; ++q)
                route[t].push_back({ (int)(((long)it * ntok * topk + t * topk + q) % E), 1.0f / topk });
        const double t0 = now();
        moe_forward(*g_pool, L, x, ntok, route, out.data(), mode);
        const double dt = now() - t0;
        if (it >= warmup) secs[it - warmup] = dt;
    }
    return 0;
}

}  // extern "C"
