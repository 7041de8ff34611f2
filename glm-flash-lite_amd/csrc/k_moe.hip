// Routed-MoE decode path on gfx950: routing plan, bit-exact trellis GEMV, activation, ordered combine.
//
// Numerics follow the reference's EXACT mode (kernels/cpu_avx2/ft_core.h:313-387, 933-1033) operation for
// operation, so outputs are bit-identical to it:
//   * each output column keeps the reference's four fp32 accumulators (AVX lanes j of tile_accum), each a chain of
//     fused multiply-adds over tile rows, and inside a tile row over the four stream groups q;
//   * the column result is (a0 + a1) + (a2 + a3);
//   * Hadamard/rounding points are those of prep_block / out_block / act_mul.
// The chain needs the weights of one (column, accumulator) in q order, while the trellis decodes four consecutive
// stream indices per lane (fixed q, accumulators 0..3). One MFMA 16x16x16 against a constant 0/1 permutation
// matrix moves the decoded tile from the first layout to the second as exact fp32 values.
#include "gfl_device.hpp"
#include "gfl_internal.hpp"

namespace gfl {

// ---------------------------------------------------------------------------------------------------------------
// routing plan
// ---------------------------------------------------------------------------------------------------------------

// One block. Picks p = t*topk + k are scanned token-major, as the reference builds its jobs
// (moe_forward, ft_core.h:1343-1349):
//   union of experts in first-appearance order (uexp), their slots (one per pick, tokens ascending), and for every
//   pick the index of the reference job it lands in (a new job whenever the expert's current job holds 8 tokens),
//   which fixes the order of the weighted sum.
// Ids outside [0, E) are skipped (tier_forward drops sel < 0, ft_tier_ext.cpp:896-898) and counted in err.
__global__ __launch_bounds__(256) void plan_kernel(const int64_t* __restrict__ sel, int P, int topk, int E, PlanView pv)
{
    __shared__ int s_e[MAX_PICKS], s_c[MAX_PICKS], s_first[MAX_PICKS], s_crank[MAX_PICKS];
    __shared__ int firstpick[MAX_EXPERTS], ucnt[MAX_PICKS], uoff[MAX_PICKS + 1];
    __shared__ int s_U, s_bad;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    for (int e = t; e < E; e += blockDim.x) firstpick[e] = 0x7fffffff;
    if (t == 0) { s_U = 0; s_bad = 0; }
    for (int p = t; p < P; p += blockDim.x)
    {
        const int64_t e = sel[p];
        s_e[p] = (e >= 0 && e < E) ? (int)e : -1;
        if (e >= E || e < -1) atomicAdd(&s_bad, 1);
        ucnt[p] = 0;
    }
    __syncthreads();
    for (int p = t; p < P; p += blockDim.x)
        if (s_e[p] >= 0) atomicMin(&firstpick[s_e[p]], p);
    // occurrence index of each pick among the picks of its expert
    for (int p = t; p < P; p += blockDim.x)
    {
        const int e = s_e[p];
        int c = 0;
        if (e >= 0)
            for (int q = 0; q < p; ++q) c += s_e[q] == e;
        s_c[p] = c;
    }
    __syncthreads();
    // wave 0: ballot prefix sums in pick order -> union rank of first picks, rank of job-creating picks
    if (wave == 0)
    {
        int base_u = 0, base_j = 0;
        for (int p0 = 0; p0 < P; p0 += 64)
        {
            const int p = p0 + lane;
            const bool ok = p < P && s_e[p] >= 0;
            const bool first = ok && s_c[p] == 0;
            const bool creator = ok && (s_c[p] % 8) == 0;
            const uint64_t mf = __ballot(first), mc = __ballot(creator);
            const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
            if (first) s_first[p] = base_u + __popcll(mf & below);
            if (creator) s_crank[p] = base_j + __popcll(mc & below);
            base_u += __popcll(mf);
            base_j += __popcll(mc);
        }
        if (lane == 0) s_U = base_u;
    }
    __syncthreads();
    const int U = s_U;
    for (int p = t; p < P; p += blockDim.x)
    {
        const int e = s_e[p];
        if (e < 0) continue;
        const int u = s_first[firstpick[e]];
        if (s_c[p] == 0) pv.uexp[u] = e;
        atomicAdd(&ucnt[u], 1);
    }
    __syncthreads();
    if (t == 0)
    {
        int acc = 0;
        for (int u = 0; u < U; ++u) { uoff[u] = acc; acc += ucnt[u]; }
        uoff[U] = acc;
        pv.hdr[0] = U;
        pv.hdr[1] = acc;
        pv.hdr[2] = s_bad;
    }
    __syncthreads();
    for (int u = t; u <= U; u += blockDim.x) pv.uoff[u] = uoff[u];
    for (int p = t; p < P; p += blockDim.x)
    {
        const int e = s_e[p];
        if (e < 0) { pv.pick_slot[p] = -1; pv.pick_job[p] = 0x7fffffff; continue; }
        const int u = s_first[firstpick[e]];
        const int slot = uoff[u] + s_c[p];
        pv.pick_slot[p] = slot;
        pv.slot_pick[slot] = p;
        pv.slot_u[slot] = u;
        // the job holding this pick was created by the pick of the same expert with occurrence 8*floor(c/8)
        const int want = (s_c[p] / 8) * 8;
        int creator = p;
        for (int q = 0; q <= p; ++q)
            if (s_e[q] == e && s_c[q] == want) { creator = q; break; }
        pv.pick_job[p] = s_crank[creator];
    }
}

// ---------------------------------------------------------------------------------------------------------------
// bit-exact trellis GEMV
// ---------------------------------------------------------------------------------------------------------------

// element r (0..127) of a 128-block -> position inside the permuted activation layout [tk][j][q] of one token:
// row rho = r % 16 of tile row tk = r / 16 is accumulator j = (rho&1) + 2*(rho>>3), group q = (rho&7)>>1
__device__ inline int perm_pos(int b, int r)
{
    const int tk = b * 8 + (r >> 4), rho = r & 15;
    const int j = (rho & 1) + 2 * (rho >> 3), q = (rho & 7) >> 1;
    return (tk * 4 + j) * 4 + q;
}

// One workgroup = 8 waves = 8 adjacent tile columns (128 outputs) of one matrix of one routed expert, all tile rows,
// for up to NS of the expert's slots at a time. Each wave owns one tile column; lane (j = l/16, n = l%16) carries the
// reference's accumulator j of output column n for every slot.
//   PREP = true : matrix is gate/up; the WG builds xt = prep_block(x_token, suh) for its slots in LDS
//   PREP = false: matrix is down; xt (already transformed and permuted) is copied from xin
template <int K, int NS, bool PREP>
__global__ __launch_bounds__(512) void chain_gemv_kernel(const uint64_t* __restrict__ ptrs, int mat_base, int kdim,
                                                         int ndim, PlanView pv, int topk,
                                                         const uint16_t* __restrict__ xin, float* __restrict__ yout)
{
    extern __shared__ uint16_t lds_x[];   // [NS][kdim] fp16, permuted [tk][j][q]
    const int TN = ndim / 16, TK = kdim / 16, ncb = TN / 8;
    const int u = blockIdx.x / ncb, cb = blockIdx.x % ncb;
    if (u >= pv.hdr[0]) return;
    const int mat = mat_base + blockIdx.y;                 // 0 gate, 1 up, 2 down
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e = pv.uexp[u];
    const uint8_t* tr = reinterpret_cast<const uint8_t*>(ptrs[(size_t)e * 9 + mat]);
    const uint16_t* suh = reinterpret_cast<const uint16_t*>(ptrs[(size_t)e * 9 + 3 + 2 * mat]);
    const int s_begin = pv.uoff[u], s_end = pv.uoff[u + 1];
    const int t = cb * 8 + wave;                           // this wave's tile column
    const LaneDec d = lane_dec(lane, K);
    const int j = lane >> 4, n = lane & 15;
    half4 Pm;
#pragma unroll
    for (int r = 0; r < 4; ++r) Pm[r] = (_Float16)((j == (n & 3) && r == (n >> 2)) ? 1.0f : 0.0f);
    const float4v zero = { 0.f, 0.f, 0.f, 0.f };
    const size_t rstride = (size_t)TN * 32 * K;
    float* ybase = yout + (size_t)blockIdx.y * (size_t)pv.cap_slots * ndim;

    for (int c0 = s_begin; c0 < s_end; c0 += NS)
    {
        const int ns = min(NS, s_end - c0);
        __syncthreads();
        if (PREP)
        {
            // xt = prep_block(x, suh) per 128-block, written permuted
            const int nb = kdim / 128;
            for (int it = wave; it < ns * nb; it += 8)
            {
                const int s = it / nb, b = it % nb;
                const int tok = pv.slot_pick[c0 + s] / topk;
                const uint16_t* xr = xin + (size_t)tok * kdim + b * 128;
                float v0 = h2f_bits(xr[lane]), v1 = h2f_bits(xr[lane + 64]);
                prep_block_wave(v0, v1, h2f_bits(suh[b * 128 + lane]), h2f_bits(suh[b * 128 + lane + 64]));
                uint16_t* dst = lds_x + (size_t)s * kdim;
                dst[perm_pos(b, lane)] = (uint16_t)f2h_bits(v0);
                dst[perm_pos(b, lane + 64)] = (uint16_t)f2h_bits(v1);
            }
        }
        else
        {
            const int nvec = ns * kdim / 8;
            const uint4* src = reinterpret_cast<const uint4*>(xin + (size_t)c0 * kdim);
            uint4* dst = reinterpret_cast<uint4*>(lds_x);
            for (int i = threadIdx.x; i < nvec; i += blockDim.x) dst[i] = src[i];
        }
        __syncthreads();

        float acc[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) acc[s] = 0.f;
        const uint8_t* tp = tr + (size_t)t * 32 * K;
        const uint16_t* xl = lds_x + j * 4;
#pragma unroll 4
        for (int tk = 0; tk < TK; ++tk)
        {
            const uint32_t hi = ld_u32(tp + d.o0), lo = ld_u32(tp + d.o1);
            tp += rstride;
            const half4 B = decode4<K>(hi, lo, d.sh);
            const float4v c = __builtin_amdgcn_mfma_f32_16x16x16f16(Pm, B, zero, 0, 0, 0);
#pragma unroll
            for (int s = 0; s < NS; ++s)
            {
                if (s < ns)
                {
                    const half4 xv = *reinterpret_cast<const half4*>(xl + ((size_t)s * TK + tk) * 16);
                    float a = acc[s];
                    a = __builtin_fmaf(c[0], (float)xv[0], a);
                    a = __builtin_fmaf(c[1], (float)xv[1], a);
                    a = __builtin_fmaf(c[2], (float)xv[2], a);
                    a = __builtin_fmaf(c[3], (float)xv[3], a);
                    acc[s] = a;
                }
            }
        }
#pragma unroll
        for (int s = 0; s < NS; ++s)
        {
            const float a1 = __shfl(acc[s], n + 16), a2 = __shfl(acc[s], n + 32), a3 = __shfl(acc[s], n + 48);
            if (s < ns && lane < 16) ybase[(size_t)(c0 + s) * ndim + t * 16 + n] = (acc[s] + a1) + (a2 + a3);
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// gate|up -> out_block -> act -> down-input prep (fwd_phase phase 1, ft_core.h:974-991)
// ---------------------------------------------------------------------------------------------------------------

__global__ __launch_bounds__(256) void act_kernel(const uint64_t* __restrict__ ptrs, PlanView pv,
                                                  const float* __restrict__ ygu, uint16_t* __restrict__ xtd, int I,
                                                  float limit)
{
    const int nb = I / 128;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int s = item / nb, ib = item % nb;
    if (s >= pv.hdr[1]) return;
    const int e = pv.uexp[pv.slot_u[s]];
    const uint16_t* svh_g = reinterpret_cast<const uint16_t*>(ptrs[(size_t)e * 9 + 4]);
    const uint16_t* svh_u = reinterpret_cast<const uint16_t*>(ptrs[(size_t)e * 9 + 6]);
    const uint16_t* suh_d = reinterpret_cast<const uint16_t*>(ptrs[(size_t)e * 9 + 7]);
    const float* yg = ygu + (size_t)s * I + ib * 128;
    const float* yu = ygu + (size_t)pv.cap_slots * I + (size_t)s * I + ib * 128;
    float g0 = yg[lane], g1 = yg[lane + 64], u0 = yu[lane], u1 = yu[lane + 64];
    out_block_wave(g0, g1, h2f_bits(svh_g[ib * 128 + lane]), h2f_bits(svh_g[ib * 128 + lane + 64]));
    out_block_wave(u0, u1, h2f_bits(svh_u[ib * 128 + lane]), h2f_bits(svh_u[ib * 128 + lane + 64]));
    float a0 = r16(act_mul(g0, u0, limit)), a1 = r16(act_mul(g1, u1, limit));
    prep_block_wave(a0, a1, h2f_bits(suh_d[ib * 128 + lane]), h2f_bits(suh_d[ib * 128 + lane + 64]));
    uint16_t* dst = xtd + (size_t)s * I;
    dst[perm_pos(ib, lane)] = (uint16_t)f2h_bits(a0);
    dst[perm_pos(ib, lane + 64)] = (uint16_t)f2h_bits(a1);
}

// ---------------------------------------------------------------------------------------------------------------
// down out_block + weighted sum in job order (fwd_phase phases 2-3, ft_core.h:1014-1033)
// ---------------------------------------------------------------------------------------------------------------

__global__ __launch_bounds__(256) void final_kernel(const uint64_t* __restrict__ ptrs, PlanView pv,
                                                    const void* __restrict__ w, int w_half, int M, int topk,
                                                    const float* __restrict__ yd, float* __restrict__ out, int H)
{
    const int nb = H / 128;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int tkn = item / nb, hb = item % nb;
    if (tkn >= M) return;
    // this token's picks sorted by (job, pick index): insertion sort of <= MAX_TOPK entries
    int ord[MAX_TOPK];
    int cnt = 0;
    for (int k = 0; k < topk; ++k)
    {
        const int p = tkn * topk + k;
        if (pv.pick_slot[p] < 0) continue;
        int b = cnt++;
        const int jb = pv.pick_job[p];
        while (b > 0 && pv.pick_job[ord[b - 1]] > jb) { ord[b] = ord[b - 1]; --b; }
        ord[b] = p;
    }
    float o0 = 0.f, o1 = 0.f;
    for (int i = 0; i < cnt; ++i)
    {
        const int p = ord[i], s = pv.pick_slot[p];
        const int e = pv.uexp[pv.slot_u[s]];
        const uint16_t* svh_d = reinterpret_cast<const uint16_t*>(ptrs[(size_t)e * 9 + 8]);
        const float wt = w_half ? h2f_bits(reinterpret_cast<const uint16_t*>(w)[p]) : reinterpret_cast<const float*>(w)[p];
        float y0 = yd[(size_t)s * H + hb * 128 + lane], y1 = yd[(size_t)s * H + hb * 128 + lane + 64];
        out_block_wave(y0, y1, h2f_bits(svh_d[hb * 128 + lane]), h2f_bits(svh_d[hb * 128 + lane + 64]));
        o0 = o0 + wt * y0;
        o1 = o1 + wt * y1;
    }
    out[(size_t)tkn * H + hb * 128 + lane] = o0;
    out[(size_t)tkn * H + hb * 128 + lane + 64] = o1;
}

// ---------------------------------------------------------------------------------------------------------------
// dequant (dense_weights, ft_core.h:1657-1672): trellis -> fp16 W[k][n]
// ---------------------------------------------------------------------------------------------------------------

template <int K>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ tr, int k, int n,
                                                      uint16_t* __restrict__ W)
{
    const int TN = n / 16, ntiles = (k / 16) * TN;
    const int tile = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (tile >= ntiles) return;
    const int tk = tile / TN, tn = tile % TN;
    const LaneDec d = lane_dec(lane, K);
    const uint8_t* tp = tr + (size_t)tile * 32 * K;
    const half4 w = decode4<K>(ld_u32(tp + d.o0), ld_u32(tp + d.o1), d.sh);
    const int q = lane >> 4, c = lane & 15;
    const int off[4] = { 0, 1, 8, 9 };
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
    {
        const int row = tk * 16 + 2 * q + off[jj];
        const _Float16 v = w[jj];
        __builtin_memcpy(&W[(size_t)row * n + tn * 16 + c], &v, 2);
    }
}

// ---------------------------------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------------------------------

void launch_plan(const int64_t* sel, int P, int topk, int E, const PlanView& pv, hipStream_t st)
{
    hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(256), 0, st, sel, P, topk, E, pv);
}

template <int K, int NS, bool PREP>
static void chain_launch(const uint64_t* ptrs, int mat_base, int nmat, int kdim, int ndim, const PlanView& pv,
                         int topk, int umax, const uint16_t* xin, float* yout, hipStream_t st)
{
    const int ncb = ndim / 128;
    const size_t lds = (size_t)NS * kdim * 2;
    auto kern = chain_gemv_kernel<K, NS, PREP>;
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(kern, dim3(umax * ncb, nmat), dim3(512), lds, st, ptrs, mat_base, kdim, ndim, pv, topk, xin,
                       yout);
}

template <int K, bool PREP>
static void chain_ns(int ns, const uint64_t* ptrs, int mat_base, int nmat, int kdim, int ndim, const PlanView& pv,
                     int topk, int umax, const uint16_t* xin, float* yout, hipStream_t st)
{
    if (ns <= 1) chain_launch<K, 1, PREP>(ptrs, mat_base, nmat, kdim, ndim, pv, topk, umax, xin, yout, st);
    else if (ns <= 2) chain_launch<K, 2, PREP>(ptrs, mat_base, nmat, kdim, ndim, pv, topk, umax, xin, yout, st);
    else if (ns <= 4) chain_launch<K, 4, PREP>(ptrs, mat_base, nmat, kdim, ndim, pv, topk, umax, xin, yout, st);
    else chain_launch<K, 8, PREP>(ptrs, mat_base, nmat, kdim, ndim, pv, topk, umax, xin, yout, st);
}

int launch_chain(int K, int ns, bool prep, const uint64_t* ptrs, int mat_base, int nmat, int kdim, int ndim,
                 const PlanView& pv, int topk, int umax, const uint16_t* xin, float* yout, hipStream_t st)
{
#define GFL_K(KK)                                                                                              \
    case KK:                                                                                                   \
        if (prep) chain_ns<KK, true>(ns, ptrs, mat_base, nmat, kdim, ndim, pv, topk, umax, xin, yout, st);     \
        else chain_ns<KK, false>(ns, ptrs, mat_base, nmat, kdim, ndim, pv, topk, umax, xin, yout, st);         \
        return 0;
    switch (K)
    {
        GFL_K(2) GFL_K(3) GFL_K(4) GFL_K(5)
        default: return -1;
    }
#undef GFL_K
}

void launch_act(const uint64_t* ptrs, const PlanView& pv, int smax, const float* ygu, uint16_t* xtd, int I,
                float limit, hipStream_t st)
{
    const int items = smax * (I / 128);
    hipLaunchKernelGGL(act_kernel, dim3((items + 3) / 4), dim3(256), 0, st, ptrs, pv, ygu, xtd, I, limit);
}

void launch_final(const uint64_t* ptrs, const PlanView& pv, const void* w, int w_half, int M, int topk,
                  const float* yd, float* out, int H, hipStream_t st)
{
    const int items = M * (H / 128);
    hipLaunchKernelGGL(final_kernel, dim3((items + 3) / 4), dim3(256), 0, st, ptrs, pv, w, w_half, M, topk, yd, out,
                       H);
}

int launch_dequant(const uint8_t* tr, int k, int n, int K, uint16_t* W, hipStream_t st)
{
    const int ntiles = (k / 16) * (n / 16);
    const dim3 g((ntiles + 3) / 4), b(256);
    switch (K)
    {
        case 2: hipLaunchKernelGGL(dequant_kernel<2>, g, b, 0, st, tr, k, n, W); return 0;
        case 3: hipLaunchKernelGGL(dequant_kernel<3>, g, b, 0, st, tr, k, n, W); return 0;
        case 4: hipLaunchKernelGGL(dequant_kernel<4>, g, b, 0, st, tr, k, n, W); return 0;
        case 5: hipLaunchKernelGGL(dequant_kernel<5>, g, b, 0, st, tr, k, n, W); return 0;
        default: return -1;
    }
}

}  // namespace gfl
