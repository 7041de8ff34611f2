// Token split / combine around the experts, plus the synthetic trellis generator.
//
// split   = ft_split (kernels/cpu_avx2/ft_tier_cu.cu:21-157 stock, kernels/k110/ft_split_fast.cu:18-198 fast):
//           count each local expert's picks (w != 0), hits = slotof[e] >= 0, rank the misses coldest first
//           (score ascending, id ascending), choose how many go to the host lane with the cost model, publish the host
//           job (x rows, picks in pick order, control words) and mask those picks out of the selection.
//           Unique experts are discovered from the picks and ranked in parallel, the cost search stays serial with the
//           reference's float expressions (uncontracted), and the published pick list is built in pick order from a
//           wavefront ballot prefix.
// combine = ft_combine (ft_tier_cu.cu:205-235, trellis build): wait (bounded) for the host done flag, add the fp32
//           partial into the fp32/fp16 output.
#include "gfl_device.hpp"
#include "gfl_internal.hpp"

namespace gfl {

__global__ __launch_bounds__(256) void split_kernel(const int64_t* __restrict__ sel, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ z, int n, int bsz, int topk, int H, int E, int first,
    const int32_t* __restrict__ slotof, const float* __restrict__ score, const float* __restrict__ p, int64_t* ctrl,
    uint16_t* hx, int32_t* hpicks, int64_t seq, int li, int keep_ids, int64_t* sel_out, uint16_t* w_out,
    int64_t* dflag, int64_t* stats, const int32_t* __restrict__ rres)
{
    __shared__ int cnt[MAX_EXPERTS];
    __shared__ unsigned char cpu[MAX_EXPERTS];
    __shared__ int s_le[MAX_PICKS];          // local expert id of pick s, or -1 (out of range)
    __shared__ unsigned char s_nz[MAX_PICKS];
    __shared__ int uq[MAX_PICKS], nu;         // unique local experts with a nonzero pick
    __shared__ int ue[MAX_PICKS];             // unique experts sorted ascending
    __shared__ int miss[MAX_PICKS], rmiss[MAX_PICKS];
    __shared__ int s_nm, s_nh, s_nr, s_publish, s_npk;
    __shared__ float pol[20];
    const int t = threadIdx.x, lane = t & 63;
    for (int e = t; e < E; e += blockDim.x) { cnt[e] = 0; cpu[e] = 0; }
    if (t < 20) pol[t] = p[t];
    if (t == 0) nu = 0;
    for (int s = t; s < n; s += blockDim.x)
    {
        const int64_t e = sel[s] - first;
        s_le[s] = (e >= 0 && e < E) ? (int)e : -1;
        s_nz[s] = (w[s] & 0x7FFFu) != 0;    // __half2float(w) != 0.0f (NaN counts as nonzero)
    }
    __syncthreads();
    for (int s = t; s < n; s += blockDim.x)
        if (s_nz[s] && s_le[s] >= 0)
            if (atomicAdd(&cnt[s_le[s]], 1) == 0) uq[atomicAdd(&nu, 1)] = s_le[s];
    __syncthreads();
    const int U = nu;
    for (int i = t; i < U; i += blockDim.x)
    {
        int r = 0;
        for (int k = 0; k < U; ++k) r += uq[k] < uq[i];
        ue[r] = uq[i];
    }
    __syncthreads();
    const bool tri = pol[8] > 0.5f && rres != nullptr && (int)pol[6] < 0;
    // misses ranked inside their class (score ascending, ties by ascending id) = the stock insertion order
    for (int i = t; i < U; i += blockDim.x)
    {
        const int e = ue[i];
        if (slotof[e] >= 0) continue;
        const int cl = (tri && rres[e]) ? 1 : 0;
        const float sc = score[e];
        int r = 0;
        for (int k = 0; k < U; ++k)
        {
            const int e2 = ue[k];
            if (slotof[e2] >= 0 || ((tri && rres[e2]) ? 1 : 0) != cl) continue;
            const float s2 = score[e2];
            if (s2 < sc || (s2 == sc && e2 < e)) ++r;
        }
        if (cl) rmiss[r] = e; else miss[r] = e;
    }
    if (t == 0)
    {
        int nh = 0, nr = 0;
        for (int i = 0; i < U; ++i)
        {
            const int e = ue[i];
            if (slotof[e] >= 0) ++nh;
            else if (tri && rres[e]) ++nr;
        }
        s_nh = nh; s_nr = nr; s_nm = U - nh - nr;
    }
    __syncthreads();
    if (t == 0)
    {
        const int nm = s_nm, nh = s_nh, nr = s_nr;
        const bool lut = pol[12] > 0.0f;
        int best = 0, bestr = 0;
        const int force = (int)pol[6], maxc = min((int)pol[5], nm);
        if (force >= 0) best = min(force, nm);
        else if (tri)
        {
            float bt = 1e30f, cr = 0.0f;
            for (int kr = 0; kr <= nr; ++kr)
            {
                if (kr) { const float f = pol[4] * (float)(cnt[rmiss[kr - 1]] - 1); const float g = 1.0f + f; cr = cr + pol[10] * g; }
                const float rem = kr ? pol[9] + cr : 0.0f;
                float c = 0.0f, cx = 0.0f;
                for (int k = 0; k <= maxc; ++k)
                {
                    if (k)
                    {
                        const float f = pol[4] * (float)(cnt[miss[k - 1]] - 1); const float g = 1.0f + f;
                        c = c + pol[3] * g;
                        const float f2 = pol[3] * pol[4];
                        cx = cx + f2 * (float)(cnt[miss[k - 1]] - 1);
                    }
                    const int zz = nm - k + nr - kr;
                    const float gpu = pol[1] * (float)(nh + zz) + pol[0] * (float)zz;
                    float loc = 0.0f;
                    if (k) loc = lut ? (pol[11 + (k < 8 ? k : 8)] + (k > 8 ? pol[3] * (float)(k - 8) : 0.0f)) + cx : pol[2] + c;
                    const float tt = fmaxf(gpu, fmaxf(loc, rem));
                    if (tt < bt - 1e-6f) { bt = tt; best = k; bestr = kr; }
                }
            }
            for (int k = 0; k < bestr; ++k) cpu[rmiss[k]] = 1;
        }
        else
        {
            float bt = 1e30f, c = 0.0f, cx = 0.0f;
            for (int k = 0; k <= maxc; ++k)
            {
                if (k)
                {
                    const float f = pol[4] * (float)(cnt[miss[k - 1]] - 1); const float g = 1.0f + f;
                    c = c + pol[3] * g;
                    const float f2 = pol[3] * pol[4];
                    cx = cx + f2 * (float)(cnt[miss[k - 1]] - 1);
                }
                const float gpu = pol[1] * (float)(nh + nm - k) + pol[0] * (float)(nm - k);
                float loc = 0.0f;
                if (k) loc = lut ? (pol[11 + (k < 8 ? k : 8)] + (k > 8 ? pol[3] * (float)(k - 8) : 0.0f)) + cx : pol[2] + c;
                const float tt = fmaxf(gpu, loc);
                if (tt < bt - 1e-6f) { bt = tt; best = k; }
            }
        }
        for (int k = 0; k < best; ++k) cpu[miss[k]] = 1;
        s_publish = best + bestr > 0 || pol[7] > 0.5f;
        stats[0] += nh; stats[1] += nm + nr; stats[2] += best + bestr; stats[3] += 1;
    }
    __syncthreads();
    const int publish = s_publish;
    if (publish && t < 64)
    {
        int base = 0;
        for (int s0 = 0; s0 < n; s0 += 64)
        {
            const int s = s0 + lane;
            const bool take = s < n && s_le[s] >= 0 && cpu[s_le[s]] && s_nz[s];
            const uint64_t m = __ballot(take);
            if (take)
            {
                const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
                const int k = base + __popcll(m & below);
                const float wf = h2f_bits(w[s]);
                int wb;
                __builtin_memcpy(&wb, &wf, 4);
                hpicks[k * 3] = s / topk;
                hpicks[k * 3 + 1] = s_le[s];
                hpicks[k * 3 + 2] = wb;
            }
            base += __popcll(m);
        }
        if (t == 0) s_npk = base;
    }
    for (int s = t; s < n; s += blockDim.x)
    {
        const int64_t e = sel[s];
        const bool c = s_le[s] >= 0 && cpu[s_le[s]];
        sel_out[s] = (c && !keep_ids) ? -1 : e;
        w_out[s] = c ? (uint16_t)0 : w[s];
    }
    if (publish)
    {
        const int nx = bsz * H / 8;
        for (int i = t; i < nx; i += blockDim.x)
            reinterpret_cast<uint4*>(hx)[i] = reinterpret_cast<const uint4*>(z)[i];
        __threadfence_system();
        __syncthreads();
        if (t == 0)
        {
            ctrl[2] = li; ctrl[3] = bsz; ctrl[4] = s_npk;
            __threadfence_system();
            __hip_atomic_store(&ctrl[0], seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
            __threadfence_system();
            dflag[0] = seq;
        }
    }
    else if (t == 0) dflag[0] = 0;
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
// router: sigmoid scores, top-k (lower index on ties), weights renormalised over the picks and rounded to fp16
// ---------------------------------------------------------------------------------------------------------------

// The router feeding ft_split (cpu_tier.py:305-307 calls the model's routing_fn, exllamav3's, which returns sel int64
// [bsz, 8] and w fp16 [bsz, 8]). One wave per token. The score is s = 1 / (1 + e) in fp32 with e = exp(-x) rounded once
// to fp32 (evaluated in double, so it is the correctly rounded value). k rounds of a wave arg-max over the unused
// experts, ordered by (score descending, index ascending); the picks' scores are summed in pick order and w_j = s_j / sum
// is rounded to fp16 (round to nearest even). Logits must be finite.
// one butterfly step of the (score descending, index ascending) arg-max: combine with lane ^ W
template <int W>
__device__ __forceinline__ void route_argmax_step(float& bv, int& bi)
{
    const float ov = lane_xor<W>(bv);
    const int oi = __float_as_int(lane_xor<W>(__int_as_float(bi)));
    if (oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi)))
    {
        bv = ov;
        bi = oi;
    }
}

constexpr int ROUTE_WAVES = 4;
constexpr int ROUTE_MAXE = 1024;   // experts per token: up to 16 per lane

// NI = ceil(E / 64) scores per lane, a compile-time count so that the per-lane loops hold only live experts
template <int NI>
__global__ __launch_bounds__(ROUTE_WAVES * 64) void route_kernel(const float* __restrict__ logits, int M, int E, int topk,
                                                                 int64_t* __restrict__ sel, uint16_t* __restrict__ w)
{
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * ROUTE_WAVES + (threadIdx.x >> 6);
    if (m >= M) return;
    const float* lg = logits + (size_t)m * E;
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
    uint32_t used = 0;
    float tot = 0.0f, mine = 0.0f;
    int myidx = 0;
    for (int j = 0; j < topk; ++j)
    {
        // this lane's best unused (score descending, index ascending: the first strict maximum in index order)
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < NI; ++i)
        {
            const int e = lane + 64 * i;
            if (e < E && !((used >> i) & 1) && (sc[i] > bv || bi == 0x7fffffff))
            {
                bv = sc[i];
                bi = e;
            }
        }
        // wave arg-max with the same order, through DPP / permlane exchanges (no LDS round trips)
        route_argmax_step<1>(bv, bi);
        route_argmax_step<2>(bv, bi);
        route_argmax_step<4>(bv, bi);
        route_argmax_step<8>(bv, bi);
        route_argmax_step<16>(bv, bi);
        route_argmax_step<32>(bv, bi);
        if ((bi & 63) == lane) used |= 1u << (bi >> 6);
        tot = tot + bv;               // pick order, as the reference's renormalisation loop
        if (lane == j)
        {
            mine = bv;
            myidx = bi;
        }
    }
    if (lane < topk)
    {
        sel[(size_t)m * topk + lane] = myidx;
        w[(size_t)m * topk + lane] = (uint16_t)f2h_bits(mine / tot);
    }
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

int launch_split(const int64_t* sel, const uint16_t* w, const uint16_t* z, int n, int bsz, int topk, int H, int E,
                 int first, const int32_t* slotof, const float* score, const float* pol, int64_t* ctrl, uint16_t* hx,
                 int32_t* hpicks, int64_t seq, int li, int keep_ids, int64_t* sel_out, uint16_t* w_out,
                 int64_t* dflag, int64_t* stats, const int32_t* rres, hipStream_t st)
{
    hipLaunchKernelGGL(split_kernel, dim3(1), dim3(256), 0, st, sel, w, z, n, bsz, topk, H, E, first, slotof, score,
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
