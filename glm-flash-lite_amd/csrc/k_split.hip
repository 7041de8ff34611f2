// Token split / combine around the experts, the router, and the synthetic trellis generator.
//
// split   = ft_split (kernels/cpu_avx2/ft_tier_cu.cu:21-157): each local expert's picks with a nonzero weight are
//           counted, resident experts (slotof[e] >= 0) are hits, the misses are ranked coldest first (score
//           ascending, id ascending), the cost model chooses how many go to the host lane, the host job is published
//           (x rows, picks in pick order, control words) and those picks leave the selection. Outputs are
//           bit-identical to the reference's; the kernel is organised for one workgroup on gfx950 (below).
// combine = ft_combine (ft_tier_cu.cu:159-236): bounded wait for the host's done word, then out += hout.
#include "gfl_device.hpp"
#include "gfl_internal.hpp"

namespace gfl {

constexpr int SP_T = 256;                 // threads of the split workgroup (4 waves)
constexpr int SP_PER = MAX_PICKS / SP_T;  // picks per thread in the pick-order scan

// LDS of the split. Experts are local ids (sel - first), picks p = token * topk + k.
struct SplitLds
{
    short le[MAX_PICKS];            // local expert of pick p, -1 outside [0, E)
    unsigned char nz[MAX_PICKS];    // weight of pick p nonzero (a NaN counts as nonzero, as __half2float(w) != 0)
    unsigned char seen[MAX_EXPERTS];
    unsigned char take[MAX_EXPERTS];   // expert goes to the host lane
    int cnt[MAX_EXPERTS];           // picks with a nonzero weight per routed expert
    int ulist[MAX_EXPERTS];         // routed experts, first-appearance order
    unsigned long long key[MAX_EXPERTS];   // sort keys of the routed experts (misses first, coldest first)
    int nu, nh, nm, nr, best, bestr, publish, npk, fast;
    int wsum[SP_T / 64];
    float pol[20];
    int slot[MAX_EXPERTS];          // the layer's residency row (slotof), loaded before the routed experts are known
    long long st[4];                // stats[0..3] before this call
    long long rsel[MAX_PICKS];      // the picks as the fused router wrote them (route_split_kernel)
    unsigned short rw[MAX_PICKS];
};

// Ascending order of finite floats as unsigned integers (+0 and -0 compare equal, as the reference's float compare
// treats them, so both map to the key of +0).
__device__ inline uint32_t float_order_key(float f)
{
    uint32_t u = __float_as_uint(f == 0.0f ? 0.0f : f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Cost model of the host lane (ft_tier_cu.cu:84-131): the reference's float expressions, each operation rounded in
// source order (this translation unit is compiled with -ffp-contract=off). miss / rmiss: local and remote misses,
// coldest first; returns best (local count) and bestr (remote count).
__device__ void split_cost(const SplitLds& S, const int* miss, const int* rmiss, int nm, int nh, int nr, bool tri,
                           int& best, int& bestr)
{
    const float* p = S.pol;
    const bool lut = p[12] > 0.0f;
    const int force = (int)p[6], maxc = min((int)p[5], nm);
    best = 0;
    bestr = 0;
    // CPU-lane time for k local experts, given the running sums c (per-expert cost) and cx (extra-token cost)
    auto lane_cpu = [&](int k, float c, float cx) -> float {
        if (!k) return 0.0f;
        if (!lut) return p[2] + c;
        const float tail = k > 8 ? p[3] * (float)(k - 8) : 0.0f;
        return (p[11 + (k < 8 ? k : 8)] + tail) + cx;
    };
    if (force >= 0)
    {
        best = min(force, nm);
        return;
    }
    const int nrr = tri ? nr : 0;
    float bt = 1e30f, cr = 0.0f;
    for (int kr = 0; kr <= nrr; ++kr)
    {
        if (kr)
        {
            const float extra = p[4] * (float)(S.cnt[rmiss[kr - 1]] - 1);
            const float one = 1.0f + extra;
            cr = cr + p[10] * one;
        }
        const float rem = kr ? p[9] + cr : 0.0f;
        float c = 0.0f, cx = 0.0f;
        for (int k = 0; k <= maxc; ++k)
        {
            if (k)
            {
                const int extra_tok = S.cnt[miss[k - 1]] - 1;
                const float one = 1.0f + p[4] * (float)extra_tok;
                c = c + p[3] * one;
                const float per = p[3] * p[4];
                cx = cx + per * (float)extra_tok;
            }
            const int zc = nm - k + nrr - kr;   // misses left to the zero-copy path
            const float gpu = p[1] * (float)(nh + zc) + p[0] * (float)zc;
            const float loc = lane_cpu(k, c, cx);
            const float tt = tri ? fmaxf(gpu, fmaxf(loc, rem)) : fmaxf(gpu, loc);
            if (tt < bt - 1e-6f)
            {
                bt = tt;
                best = k;
                bestr = kr;
            }
        }
    }
}

// The split of one call (whole workgroup). sel/w are read from global memory (the caller's selection, or the router
// output written by this workgroup before a barrier).
// PRE: the fused router already put the picks (S.rsel, S.rw), the residency row (S.slot), the policy (S.pol) and
// stats[0..3] (S.st) in LDS; else they are loaded here, all in one round trip.
template <bool PRE>
__device__ void split_body(SplitLds& S, const int64_t* __restrict__ sel, const uint16_t* __restrict__ w,
                           const uint16_t* __restrict__ z, int n, int bsz, int topk, int H, int E, int first,
                           const int32_t* __restrict__ slotof, const float* __restrict__ score,
                           const float* __restrict__ pol, int64_t* ctrl, uint16_t* hx, int32_t* hpicks, int64_t seq,
                           int li, int keep_ids, int64_t* sel_out, uint16_t* w_out, int64_t* dflag, int64_t* stats,
                           const int32_t* __restrict__ rres)
{
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    // 1. per-pick classification
    if (!PRE)
    {
        for (int q = t; q < n; q += SP_T)
        {
            S.rsel[q] = sel[q];
            S.rw[q] = w[q];
        }
        for (int e = t; e < E; e += SP_T) S.slot[e] = slotof[e];
        if (t < 4) S.st[t] = stats[t];
        if (t < 20) S.pol[t] = pol[t];
        __syncthreads();
    }
    // decode calls at full residency (the common case): with at most 64 picks, every routed expert resident and no
    // handshake policy, nothing goes to the host lane and the split is the identity plus the hit count. One wave
    // decides it from registers (lane = pick); the phases below, each ending in a barrier, measured 3.3 us of the
    // fused router + split at M = 1..4 for what this does in about one.
    if (n <= 64 && !(S.pol[7] > 0.5f))
    {
        if (wv == 0)
        {
            const int64_t e64 = lane < n ? S.rsel[lane] - first : -1;
            const bool ok = lane < n && e64 >= 0 && e64 < E && (S.rw[lane] & 0x7FFFu) != 0;
            const int e = ok ? (int)e64 : 0;
            uint64_t eq = __ballot(ok);
#pragma unroll
            for (int b = 0; b < 10; ++b)
            {
                const bool bit = ok && ((e >> b) & 1);
                const uint64_t m = __ballot(bit);
                eq &= bit ? m : ~m;
            }
            const bool leader = ok && (int)__builtin_ctzll(eq) == lane;   // one lane per routed expert
            const bool hit = leader && S.slot[e] >= 0;
            const uint64_t mh = __ballot(hit), mm = __ballot(leader && !hit);
            if (lane == 0)
            {
                S.fast = mm == 0;
                S.nh = __popcll(mh);
            }
        }
        __syncthreads();
        if (S.fast)
        {
            for (int q = t; q < n; q += SP_T)
            {
                sel_out[q] = S.rsel[q];
                w_out[q] = S.rw[q];
            }
            if (t == 0)
            {
                stats[0] = S.st[0] + S.nh;
                stats[1] = S.st[1];
                stats[2] = S.st[2];
                stats[3] = S.st[3] + 1;
                dflag[0] = 0;
            }
            return;
        }
    }
    for (int q = t; q < n; q += SP_T)
    {
        const int64_t e = S.rsel[q] - first;
        S.le[q] = (e >= 0 && e < E) ? (short)e : (short)-1;
        S.nz[q] = (S.rw[q] & 0x7FFFu) != 0;
    }
    for (int e = t; e < E; e += SP_T) { S.seen[e] = 0; S.take[e] = 0; }
    if (t == 0) { S.nh = 0; S.nm = 0; S.nr = 0; }
    __syncthreads();
    // 2. routed experts in first-appearance order, and their nonzero-pick counts (wave 0)
    if (wv == 0)
    {
        int nu = 0;
        for (int q0 = 0; q0 < n; q0 += 64)
        {
            const int q = q0 + lane;
            const int e = (q < n && S.nz[q]) ? S.le[q] : -1;
            const bool ok = e >= 0;
            uint64_t eq = __ballot(ok);
#pragma unroll
            for (int b = 0; b < 10; ++b)
            {
                const bool bit = ok && ((e >> b) & 1);
                const uint64_t m = __ballot(bit);
                eq &= bit ? m : ~m;
            }
            const bool leader = ok && (int)__builtin_ctzll(eq) == lane;   // lowest lane of its expert in the chunk
            const bool fresh = leader && !S.seen[e];
            if (leader)
            {
                S.cnt[e] = (fresh ? 0 : S.cnt[e]) + __popcll(eq);
                S.seen[e] = 1;
            }
            const uint64_t mf = __ballot(fresh);
            if (fresh) S.ulist[nu + __popcll(mf & below)] = e;
            nu += __popcll(mf);
        }
        if (lane == 0) S.nu = nu;
    }
    __syncthreads();
    const int U = S.nu;
    const bool tri = S.pol[8] > 0.5f && rres != nullptr && (int)S.pol[6] < 0;
    // 3. classes and sort keys: local miss (key bit 63 clear), remote miss (set), hit (all ones, sorted last)
    int h = 0, ml = 0, mr = 0;
    for (int i = t; i < U; i += SP_T)
    {
        const int e = S.ulist[i];
        unsigned long long k = ~0ull;
        if (S.slot[e] >= 0) ++h;
        else
        {
            const bool remote = tri && rres[e];
            remote ? ++mr : ++ml;
            k = ((unsigned long long)remote << 63) | ((unsigned long long)float_order_key(score[e]) << 31) |
                (unsigned long long)e;
        }
        S.key[i] = k;
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1)
    {
        h += __shfl_xor(h, d);
        ml += __shfl_xor(ml, d);
        mr += __shfl_xor(mr, d);
    }
    if (lane == 0)
    {
        atomicAdd(&S.nh, h);
        atomicAdd(&S.nm, ml);
        atomicAdd(&S.nr, mr);
    }
    __syncthreads();
    const int nh = S.nh, nm = S.nm, nr = S.nr;
    // 4. coldest-first order of the misses: one bitonic sort of the keys (unique: the id is part of the key)
    if (nm + nr > 0)
    {
        int N = 1;
        while (N < U) N <<= 1;
        for (int i = U + t; i < N; i += SP_T) S.key[i] = ~0ull;
        __syncthreads();
        for (int k = 2; k <= N; k <<= 1)
            for (int j = k >> 1; j > 0; j >>= 1)
            {
                for (int i = t; i < N; i += SP_T)
                {
                    const int o = i ^ j;
                    if (o > i)
                    {
                        const unsigned long long a = S.key[i], b = S.key[o];
                        if ((a > b) == ((i & k) == 0))
                        {
                            S.key[i] = b;
                            S.key[o] = a;
                        }
                    }
                }
                __syncthreads();
            }
        // keys -> expert ids in place (miss list then remote list), for the cost model
        for (int i = t; i < nm + nr; i += SP_T) S.ulist[i] = (int)(S.key[i] & 0x7FFFFFFFull);
        __syncthreads();
    }
    // 5. cost model (one thread), host-lane flags, stats
    if (t == 0)
    {
        int best = 0, bestr = 0;
        if (nm + nr > 0) split_cost(S, S.ulist, S.ulist + nm, nm, nh, nr, tri, best, bestr);
        for (int k = 0; k < best; ++k) S.take[S.ulist[k]] = 1;
        for (int k = 0; k < bestr; ++k) S.take[S.ulist[nm + k]] = 1;
        S.best = best;
        S.bestr = bestr;
        S.publish = best + bestr > 0 || S.pol[7] > 0.5f;
        stats[0] = S.st[0] + nh;
        stats[1] = S.st[1] + nm + nr;
        stats[2] = S.st[2] + best + bestr;
        stats[3] = S.st[3] + 1;
    }
    __syncthreads();
    const bool publish = S.publish, any_taken = S.best + S.bestr > 0;
    // 6. selection for the device experts, and the host job's picks in pick order (a workgroup exclusive scan over
    // per-thread runs of SP_PER consecutive picks)
    for (int q = t; q < n; q += SP_T)
    {
        const int e = S.le[q];
        const bool c = e >= 0 && S.take[e];
        sel_out[q] = (c && !keep_ids) ? -1 : S.rsel[q];
        w_out[q] = c ? (uint16_t)0 : S.rw[q];
    }
    if (publish)
    {
        int mine = 0;
        const int q0 = t * SP_PER;
        if (any_taken)
            for (int i = 0; i < SP_PER; ++i)
            {
                const int q = q0 + i;
                mine += (q < n && S.le[q] >= 0 && S.take[S.le[q]] && S.nz[q]) ? 1 : 0;
            }
        int incl = mine;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1)
        {
            const int o = __shfl_up(incl, d);
            if (lane >= d) incl += o;
        }
        if (lane == 63) S.wsum[wv] = incl;
        __syncthreads();
        int base = incl - mine;
        for (int v = 0; v < wv; ++v) base += S.wsum[v];
        if (t == SP_T - 1) S.npk = base + mine;
        for (int i = 0; i < SP_PER && mine; ++i)
        {
            const int q = q0 + i;
            if (q < n && S.le[q] >= 0 && S.take[S.le[q]] && S.nz[q])
            {
                hpicks[base * 3] = q / topk;
                hpicks[base * 3 + 1] = S.le[q];
                hpicks[base * 3 + 2] = (int32_t)__float_as_uint(h2f_bits(S.rw[q]));
                ++base;
            }
        }
        // x rows of the job, then the control words (the sequence number last, system scope, for the host reader)
        const int nx = bsz * H / 8;
        for (int i = t; i < nx; i += SP_T) reinterpret_cast<uint4*>(hx)[i] = reinterpret_cast<const uint4*>(z)[i];
        __threadfence_system();
        __syncthreads();
        if (t == 0)
        {
            const int npk = S.npk;
            ctrl[2] = li;
            ctrl[3] = bsz;
            ctrl[4] = npk;
            __threadfence_system();
            __hip_atomic_store(&ctrl[0], seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
            __threadfence_system();
            dflag[0] = seq;
        }
    }
    else if (t == 0) dflag[0] = 0;
}

__global__ __launch_bounds__(SP_T) void split_kernel(const int64_t* __restrict__ sel, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ z, int n, int bsz, int topk, int H, int E, int first,
    const int32_t* __restrict__ slotof, const float* __restrict__ score, const float* __restrict__ pol, int64_t* ctrl,
    uint16_t* hx, int32_t* hpicks, int64_t seq, int li, int keep_ids, int64_t* sel_out, uint16_t* w_out,
    int64_t* dflag, int64_t* stats, const int32_t* __restrict__ rres)
{
    __shared__ SplitLds S;
    split_body<false>(S, sel, w, z, n, bsz, topk, H, E, first, slotof, score, pol, ctrl, hx, hpicks, seq, li,
                      keep_ids, sel_out, w_out, dflag, stats, rres);
}

// One workgroup decides once, for every output element, whether the host partial is added: the trellis build of the
// reference waits in each of its 16 blocks separately (ft_tier_cu.cu:205-235), so a done flag that lands inside the
// timeout window can be added by some blocks and dropped by others; its LUT build already moved the decision into a
// single block (ft_tier_cu.cu:162-201). Same counters: stats[4] waited ns, [5] waits, [6] timeouts, [7] already done.
// timeout_ticks: bounded wait in wall-clock ticks (the caller converts ns with the device's wall clock rate).
__global__ __launch_bounds__(1024) void combine_kernel(void* out, int is_half, int n, const int64_t* __restrict__ dflag,
                                                       const int64_t* ctrl, const float* hout, int64_t* stats,
                                                       int64_t timeout_ticks, int64_t ns_per_tick_q16)
{
    __shared__ int go;
    if (threadIdx.x == 0)
    {
        const int64_t s = dflag[0];
        go = s != 0;
        if (go)
        {
            const int64_t* done = ctrl + 1;
            if (__hip_atomic_load(done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) >= s)
                atomicAdd(reinterpret_cast<unsigned long long*>(&stats[7]), 1ull);
            const uint64_t t0 = wall_clock64();
            uint64_t t1 = t0;
            while (__hip_atomic_load(done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) < s)
            {
                t1 = wall_clock64();
                if ((int64_t)(t1 - t0) > timeout_ticks)
                {
                    go = 0;
                    atomicAdd(reinterpret_cast<unsigned long long*>(&stats[6]), 1ull);
                    break;
                }
            }
            const unsigned long long waited = (unsigned long long)(((t1 - t0) * (uint64_t)ns_per_tick_q16) >> 16);
            atomicAdd(reinterpret_cast<unsigned long long*>(&stats[4]), waited);
            atomicAdd(reinterpret_cast<unsigned long long*>(&stats[5]), 1ull);
        }
    }
    __syncthreads();
    if (!go) return;
    for (int i = threadIdx.x; i < n; i += blockDim.x)
    {
        const float v = __hip_atomic_load(&hout[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        if (is_half)
        {
            uint16_t* o = reinterpret_cast<uint16_t*>(out);
            o[i] = (uint16_t)f2h_bits(h2f_bits(o[i]) + v);
        }
        else reinterpret_cast<float*>(out)[i] += v;
    }
}

// ---------------------------------------------------------------------------------------------------------------
// device worker: the consumer of a published job (run_job + worker_main, ft_tier_ext.cpp:400-627, 781-802)
// ---------------------------------------------------------------------------------------------------------------

// The worker's read of a published job. A job is pending when ctrl[0] (the split's sequence number) differs from
// ctrl[1] (the last one answered). It is accepted when it names layer li, ntok = ctrl[3] <= bsz tokens and
// np = ctrl[4] <= ntok * topk picks, each pick (token, expert, weight bits) with a token in [0, ntok), an expert in
// [0, E) and at most topk picks per token (run_job indexes its route and the layer with them unchecked). Its picks
// are laid out as a selection sel int64 [bsz][topk] / w fp32 [bsz][topk]: token t's picks in pick order, then -1 / 0.
// That is run_job's route[t] (picks pushed in pick order), which moe_forward walks token-major, so the forward on
// this selection builds the reference's jobs in the reference's order. No pending job, or a refused one: the
// selection stays empty (a refused job counts in status[GFL_STATUS_INGRESS_REJECTED] and is never answered, so the
// combine waits out its timeout and counts it). state = {1 if accepted, the job's sequence number}.
__global__ __launch_bounds__(256) void ingress_take_kernel(const int64_t* ctrl, const int32_t* hpicks, int li, int bsz,
                                                           int topk, int E, int64_t* sel, float* w, int64_t* state,
                                                           int* status)
{
    __shared__ int s_job, s_ntok, s_np, s_bad;
    __shared__ int64_t s_seq;
    __shared__ int pt[MAX_PICKS], pe[MAX_PICKS], pw[MAX_PICKS], cnt[MAX_PICKS];
    const int t = threadIdx.x, nt = blockDim.x, n = bsz * topk;
    for (int i = t; i < n; i += nt) { sel[i] = -1; w[i] = 0.0f; }
    for (int i = t; i < bsz; i += nt) cnt[i] = 0;
    if (t == 0)
    {
        const int64_t seq = __hip_atomic_load(&ctrl[0], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
        const int64_t done = __hip_atomic_load(&ctrl[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        const int64_t jl = __hip_atomic_load(&ctrl[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        const int64_t jt = __hip_atomic_load(&ctrl[3], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        const int64_t jp = __hip_atomic_load(&ctrl[4], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        const bool pending = seq != done;
        const bool ok = jl == li && jt >= 0 && jt <= bsz && jp >= 0 && jp <= jt * topk;
        s_job = !pending ? 0 : ok ? 1 : -1;
        s_seq = seq;
        s_ntok = ok ? (int)jt : 0;
        s_np = ok ? (int)jp : 0;
        s_bad = 0;
    }
    __syncthreads();
    const int np = s_np, ntok = s_ntok;
    if (s_job == 1)
    {
        for (int k = t; k < np; k += nt)
        {
            const int tk = hpicks[3 * k], e = hpicks[3 * k + 1];
            pt[k] = tk;
            pe[k] = e;
            pw[k] = hpicks[3 * k + 2];
            if (tk < 0 || tk >= ntok || e < 0 || e >= E) s_bad = 1;
            else if (atomicAdd(&cnt[tk], 1) >= topk) s_bad = 1;
        }
        __syncthreads();
        if (!s_bad)
            for (int tk = t; tk < ntok; tk += nt)
            {
                int c = 0;
                for (int k = 0; k < np; ++k)
                    if (pt[k] == tk)
                    {
                        sel[tk * topk + c] = pe[k];
                        w[tk * topk + c] = __int_as_float(pw[k]);
                        ++c;
                    }
            }
    }
    if (t == 0)
    {
        const bool accepted = s_job == 1 && !s_bad;
        state[0] = accepted ? 1 : 0;
        state[1] = s_seq;
        if (s_job == -1 || (s_job == 1 && s_bad))
            __hip_atomic_fetch_add(&status[GFL_STATUS_INGRESS_REJECTED], 1, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The worker's answer (worker_main, ft_tier_ext.cpp:797-799): after the forward has written hout, the done word
// ctrl[1] = the job's sequence number, released at system scope (hout first).
__global__ void ingress_answer_kernel(int64_t* ctrl, const int64_t* state)
{
    if (threadIdx.x == 0 && state[0] == 1)
    {
        __threadfence_system();
        __hip_atomic_store(&ctrl[1], state[1], __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

void launch_ingress_take(const int64_t* ctrl, const int32_t* hpicks, int li, int bsz, int topk, int E, int64_t* sel,
                         float* w, int64_t* state, int* status, hipStream_t st)
{
    hipLaunchKernelGGL(ingress_take_kernel, dim3(1), dim3(256), 0, st, ctrl, hpicks, li, bsz, topk, E, sel, w, state,
                       status);
}

void launch_ingress_answer(int64_t* ctrl, const int64_t* state, hipStream_t st)
{
    hipLaunchKernelGGL(ingress_answer_kernel, dim3(1), dim3(64), 0, st, ctrl, state);
}

// ---------------------------------------------------------------------------------------------------------------
// router: sigmoid scores, top-k (lower index on ties), weights renormalised over the picks and rounded to fp16
// ---------------------------------------------------------------------------------------------------------------

// The router feeding ft_split (cpu_tier.py:305-307 calls the model's routing_fn, exllamav3's, which returns sel int64
// [bsz, 8] and w fp16 [bsz, 8]). One wave per token. The score is s = 1 / (1 + e) in fp32 with e = exp(-x) rounded once
// to fp32 (evaluated in double, so it is the correctly rounded value). k rounds of a wave arg-max over the unused
// experts, ordered by (score descending, index ascending); the picks' scores are summed in pick order and
// w_j = s_j / sum
// is rounded to fp16 (round to nearest even). Logits must be finite.
// One butterfly step of the wave arg-max on 64-bit keys (order-preserving score bits above the complemented index, so
// the larger key is the higher score and, on a tie, the lower index; 0 = no candidate): combine with lane ^ W.
template <int W>
__device__ __forceinline__ void route_argmax_step(uint32_t& hi, uint32_t& lo)
{
    const uint32_t ohi = __float_as_uint(lane_xor<W>(__uint_as_float(hi)));
    const uint32_t olo = __float_as_uint(lane_xor<W>(__uint_as_float(lo)));
    if ((((uint64_t)ohi << 32) | olo) > (((uint64_t)hi << 32) | lo))
    {
        hi = ohi;
        lo = olo;
    }
}

constexpr int ROUTE_WAVES = 4;
constexpr int ROUTE_MAXE = 1024;   // experts per token: up to 16 per lane

// One token on one wave: sel_row[0..topk) / w_row[0..topk) from logits row lg. NI = ceil(E / 64) scores per lane, a
// compile-time count so that the per-lane loops hold only live experts.
template <int NI>
__device__ __forceinline__ void route_token(const float* __restrict__ lg, int E, int topk, int64_t* sel_row,
                                            uint16_t* w_row, long long* lsel = nullptr, unsigned short* lw = nullptr)
{
    const int lane = threadIdx.x & 63;
    // every load first (uniform guards, clamped addresses), so the token's logits arrive in one round trip
    float sc[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) sc[i] = lg[min(lane + 64 * i, E - 1)];
#pragma unroll
    for (int i = 0; i < NI; ++i)
    {
        const float ex = (float)exp(-(double)sc[i]);
        sc[i] = lane + 64 * i < E ? 1.0f / (1.0f + ex) : -INFINITY;
    }
    // each candidate as a 64-bit key: the score's order-preserving bits above the complemented expert index, so that
    // the largest key is the highest score and, among equal scores, the lowest index (the reference's first strict
    // maximum in index order); a picked or absent candidate is key 0
    uint32_t khi[NI], klo[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i)
    {
        const int e = lane + 64 * i;
        khi[i] = e < E ? float_order_key(sc[i]) : 0u;
        klo[i] = e < E ? ~(uint32_t)e : 0u;
    }
    float tot = 0.0f, mine = 0.0f;
    int myidx = 0;
    for (int j = 0; j < topk; ++j)
    {
        // this lane's best remaining candidate, then the wave's, through DPP / permlane exchanges
        uint32_t hi = khi[0], lo = klo[0];
#pragma unroll
        for (int i = 1; i < NI; ++i)
            if ((((uint64_t)khi[i] << 32) | klo[i]) > (((uint64_t)hi << 32) | lo))
            {
                hi = khi[i];
                lo = klo[i];
            }
        route_argmax_step<1>(hi, lo);
        route_argmax_step<2>(hi, lo);
        route_argmax_step<4>(hi, lo);
        route_argmax_step<8>(hi, lo);
        route_argmax_step<16>(hi, lo);
        route_argmax_step<32>(hi, lo);
        const int bi = (int)~lo;
        const float bv = __uint_as_float((hi & 0x80000000u) ? (hi & 0x7FFFFFFFu) : ~hi);
#pragma unroll
        for (int i = 0; i < NI; ++i)
            if (bi == lane + 64 * i) khi[i] = klo[i] = 0u;
        tot = tot + bv;               // pick order, as the reference's renormalisation loop
        if (lane == j)
        {
            mine = bv;
            myidx = bi;
        }
    }
    if (lane < topk)
    {
        const uint16_t wb = (uint16_t)f2h_bits(mine / tot);
        sel_row[lane] = myidx;
        w_row[lane] = wb;
        if (lsel)
        {
            lsel[lane] = myidx;
            lw[lane] = wb;
        }
    }
}

template <int NI>
__global__ __launch_bounds__(ROUTE_WAVES * 64) void route_kernel(const float* __restrict__ logits, int M, int E, int topk,
                                                                 int64_t* __restrict__ sel, uint16_t* __restrict__ w)
{
    const int m = blockIdx.x * ROUTE_WAVES + (threadIdx.x >> 6);
    if (m >= M) return;
    route_token<NI>(logits + (size_t)m * E, E, topk, sel + (size_t)m * topk, w + (size_t)m * topk);
}

// Router and split in one launch (the routing_fn that cpu_tier.routed wraps, glm53/cpu_tier.py:305-333): the
// workgroup's waves route the M tokens into sel / w (kept: the caller's original selection), then the workgroup runs
// the split on them.
template <int NI>
__global__ __launch_bounds__(SP_T) void route_split_kernel(const float* __restrict__ logits, int M, int ER, int topk,
    int64_t* sel, uint16_t* w, const uint16_t* __restrict__ z, int H, int E, int first,
    const int32_t* __restrict__ slotof, const float* __restrict__ score, const float* __restrict__ pol, int64_t* ctrl,
    uint16_t* hx, int32_t* hpicks, int64_t seq, int li, int keep_ids, int64_t* sel_out, uint16_t* w_out,
    int64_t* dflag, int64_t* stats, const int32_t* __restrict__ rres)
{
    __shared__ SplitLds S;
    const int t = threadIdx.x;
    // the split's inputs that do not depend on the routing, loaded first so that their round trip overlaps the
    // logits'; the routed picks go to the split through LDS
    constexpr int SLOT_PER = (MAX_EXPERTS + SP_T - 1) / SP_T;
    int32_t slot_r[SLOT_PER];
#pragma unroll
    for (int i = 0; i < SLOT_PER; ++i) slot_r[i] = t + i * SP_T < E ? slotof[t + i * SP_T] : 0;
    const long long st_r = t < 4 ? (long long)stats[t] : 0;
    const float pol_r = t < 20 ? pol[t] : 0.f;
    for (int m = t >> 6; m < M; m += SP_T / 64)
        route_token<NI>(logits + (size_t)m * ER, ER, topk, sel + (size_t)m * topk, w + (size_t)m * topk,
                        S.rsel + (size_t)m * topk, S.rw + (size_t)m * topk);
#pragma unroll
    for (int i = 0; i < SLOT_PER; ++i)
        if (t + i * SP_T < E) S.slot[t + i * SP_T] = slot_r[i];
    if (t < 4) S.st[t] = st_r;
    if (t < 20) S.pol[t] = pol_r;
    __syncthreads();
    split_body<true>(S, sel, w, z, M * topk, M, topk, H, E, first, slotof, score, pol, ctrl, hx, hpicks, seq, li,
                     keep_ids, sel_out, w_out, dflag, stats, rres);
}

int launch_route(const float* logits, int M, int E, int topk, int64_t* sel, uint16_t* w, hipStream_t st)
{
    if (E < 1 || E > ROUTE_MAXE || topk < 1 || topk > E || topk > 64) return -1;
    const dim3 grid((M + ROUTE_WAVES - 1) / ROUTE_WAVES), block(ROUTE_WAVES * 64);
    switch ((E + 63) / 64)
    {
#define GFL_ROUTE_CASE(N)                                                                                          \
    case N: hipLaunchKernelGGL(route_kernel<N>, grid, block, 0, st, logits, M, E, topk, sel, w); return 0;
        GFL_ROUTE_CASE(1) GFL_ROUTE_CASE(2) GFL_ROUTE_CASE(3) GFL_ROUTE_CASE(4) GFL_ROUTE_CASE(5) GFL_ROUTE_CASE(6)
        GFL_ROUTE_CASE(7) GFL_ROUTE_CASE(8) GFL_ROUTE_CASE(9) GFL_ROUTE_CASE(10) GFL_ROUTE_CASE(11) GFL_ROUTE_CASE(12)
        GFL_ROUTE_CASE(13) GFL_ROUTE_CASE(14) GFL_ROUTE_CASE(15) GFL_ROUTE_CASE(16)
#undef GFL_ROUTE_CASE
        default: return -1;
    }
}

// splitmix64 in counter form: output i of the sequence seeded with `seed` is mix(seed + (i+1) * golden)
__device__ inline uint64_t splitmix64_at(uint64_t seed, uint64_t i)
{
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void synth_kernel(uint8_t* dst, size_t nbytes, uint64_t seed)
{
    const size_t nw = nbytes / 8;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nw; i += (size_t)gridDim.x * blockDim.x)
        reinterpret_cast<uint64_t*>(dst)[i] = splitmix64_at(seed, i);
    if (blockIdx.x == 0 && threadIdx.x == 0)
    {
        const uint64_t v = splitmix64_at(seed, nw);
        for (size_t b = nw * 8; b < nbytes; ++b) dst[b] = (uint8_t)(v >> (8 * (b - nw * 8)));
    }
}

int launch_route_split(const float* logits, int M, int ER, int topk, int64_t* sel, uint16_t* w, const uint16_t* z,
                       int H, int E, int first, const int32_t* slotof, const float* score, const float* pol,
                       int64_t* ctrl, uint16_t* hx, int32_t* hpicks, int64_t seq, int li, int keep_ids,
                       int64_t* sel_out, uint16_t* w_out, int64_t* dflag, int64_t* stats, const int32_t* rres,
                       hipStream_t st)
{
    if (ER < 1 || ER > ROUTE_MAXE || topk < 1 || topk > ER || topk > 64 || M * topk > MAX_PICKS) return -1;
    // one launch while each of its waves routes at most one token. Above that its waves would take their tokens one
    // after another (one logits round trip and about 2 us of exponentials and argmax rounds each: 17.7 / 32.0 /
    // 58.9 us at M = 16 / 32 / 64), so the router runs over a grid of its own (a wave per token) and the split follows
    // as a second launch; both write what the fused launch writes, bit for bit.
    if (M > SP_T / 64)
    {
        if (launch_route(logits, M, ER, topk, sel, w, st)) return -1;
        return launch_split(sel, w, z, M * topk, M, topk, H, E, first, slotof, score, pol, ctrl, hx, hpicks, seq, li,
                            keep_ids, sel_out, w_out, dflag, stats, rres, st);
    }
    switch ((ER + 63) / 64)
    {
#define GFL_RS_CASE(N)                                                                                             \
    case N:                                                                                                        \
        hipLaunchKernelGGL(route_split_kernel<N>, dim3(1), dim3(SP_T), 0, st, logits, M, ER, topk, sel, w, z, H, E,  \
                           first, slotof, score, pol, ctrl, hx, hpicks, seq, li, keep_ids, sel_out, w_out, dflag,   \
                           stats, rres);                                                                           \
        return 0;
        GFL_RS_CASE(1) GFL_RS_CASE(2) GFL_RS_CASE(3) GFL_RS_CASE(4) GFL_RS_CASE(5) GFL_RS_CASE(6) GFL_RS_CASE(7)
        GFL_RS_CASE(8) GFL_RS_CASE(9) GFL_RS_CASE(10) GFL_RS_CASE(11) GFL_RS_CASE(12) GFL_RS_CASE(13)
        GFL_RS_CASE(14) GFL_RS_CASE(15) GFL_RS_CASE(16)
#undef GFL_RS_CASE
        default: return -1;
    }
}

int launch_split(const int64_t* sel, const uint16_t* w, const uint16_t* z, int n, int bsz, int topk, int H, int E,
                 int first, const int32_t* slotof, const float* score, const float* pol, int64_t* ctrl, uint16_t* hx,
                 int32_t* hpicks, int64_t seq, int li, int keep_ids, int64_t* sel_out, uint16_t* w_out,
                 int64_t* dflag, int64_t* stats, const int32_t* rres, hipStream_t st)
{
    hipLaunchKernelGGL(split_kernel, dim3(1), dim3(SP_T), 0, st, sel, w, z, n, bsz, topk, H, E, first, slotof, score,
                       pol, ctrl, hx, hpicks, seq, li, keep_ids, sel_out, w_out, dflag, stats, rres);
    return 0;
}

void launch_combine(void* out, int is_half, int n, const int64_t* dflag, const int64_t* ctrl, const float* hout,
                    int64_t* stats, int64_t timeout_ns, hipStream_t st)
{
    int dev = 0, khz = 100000;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0) khz = 100000;
    const int64_t ticks = (int64_t)((double)timeout_ns * (double)khz / 1e6);
    const int64_t ns_per_tick_q16 = (int64_t)(65536.0 * 1e6 / (double)khz);
    hipLaunchKernelGGL(combine_kernel, dim3(1), dim3(1024), 0, st, out, is_half, n, dflag, ctrl, hout, stats, ticks,
                       ns_per_tick_q16);
}

void launch_synth(uint8_t* dst, size_t nbytes, uint64_t seed, hipStream_t st)
{
    const size_t nw = nbytes / 8;
    size_t blocks = (nw + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) blocks = 1;
    hipLaunchKernelGGL(synth_kernel, dim3((unsigned)blocks), dim3(256), 0, st, dst, nbytes, seed);
}

}  // namespace gfl
