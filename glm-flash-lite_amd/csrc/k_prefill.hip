// Prefill-sized routed-MoE layer on gfx950: grouped rows, the input transforms, two MFMA grouped GEMMs on trellis
// tiles decoded into registers, SwiGLU, output transform and weighted combine.
//
// The decode path (k_moe.hip) reproduces the reference's EXACT accumulation order, which keeps every product in a
// sequential fp32 chain; at prefill sizes (thousands of tokens) that order is an MFMA-free GEMM. This path instead
// accumulates with v_mfma_f32_16x16x32_f16: dequantized weights are the same bit-exact fp16 values, every rounding
// point of the reference's transforms is kept (prep_block, out_block, act_mul; ft_core.h:96-132), but the sums over
// the hidden dimension are formed in MFMA order. Its outputs therefore differ from EXACT by accumulation rounding
// only, the same way the reference's own fp64 expert does (ref_expert, ft_core.h:1674-1691).
//
// Operand layout: the trellis decode leaves lane l = 16q + n holding the four weights of column n at tile rows
// 2q + {0, 1, 8, 9}. That is exactly the B slice of lane l in v_mfma_f32_16x16x16_f16 when the k index 4q + jj stands
// for tile row 2q + {0, 1, 8, 9}[jj]; the inputs are stored with the same row permutation ([tk][q][jj] per tile row),
// so each decoded tile feeds the MFMA directly, with no transpose. gfx950's v_mfma_f32_16x16x32_f16 takes two such
// slices (tile rows r and r + 1) per lane as its 8 k-values.
#include <type_traits>

#include "gfl_device.hpp"
#include "gfl_internal.hpp"

namespace gfl {

// ---------------------------------------------------------------------------------------------------------------
// grouped rows (tier_lut_build_grouped_rows semantics, ft_tier_ext.cpp:1047-1097) and the combine order
// ---------------------------------------------------------------------------------------------------------------

constexpr int GP_MT = 80;          // slots per GEMM pass (up to 5 MFMA row blocks)
constexpr int GP_PLAN_THREADS = GP_PLAN_CHUNK;   // one thread per pick of a chunk
constexpr int GP_PLAN_WAVES = GP_PLAN_THREADS / 64;
constexpr int GP_ORDER_THREADS = 256;

// Slots are expert-major, experts ascending, picks (hence tokens) ascending within an expert; picks with ids outside
// [0, E) are skipped (ids other than -1 are counted in hdr[1]). The combine order of a token's picks is the
// reference's job order: moe_forward (ft_core.h:1343-1349) scans picks token-major and opens a job for an expert at
// its first pick and after every 8 of its picks, so pick p (the c-th of its expert) lands in the job opened by that
// expert's pick number c - c % 8, and jobs are numbered in the order their opening picks appear. The plan takes three
// launches over chunks of GP_PLAN_CHUNK picks: ranks within each chunk, then placement (every chunk sums the counts
// of the chunks before it), then each token's picks in job order.

// Bit mask of the lanes below this one.
__device__ __forceinline__ uint64_t gp_lanes_below(int lane)
{
    return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Pass 1, one workgroup per chunk: each pick's rank among the same-expert picks of its chunk, in pick order (same
// expert lanes of a wave from ten ballots on the id bits, E <= 1024, plus the group sizes of the waves before), into
// pick_c; and the chunk's per-expert counts into ccnt[chunk][0, E), with its count of ids outside [-1, E) at [E].
__global__ __launch_bounds__(GP_PLAN_THREADS) void gp_rank_kernel(const int64_t* __restrict__ sel, int P, int E,
                                                                  GPlan g)
{
    __shared__ int s_cnt[MAX_EXPERTS];
    __shared__ unsigned char s_wcnt[GP_PLAN_WAVES][MAX_EXPERTS];   // group sizes (<= 64) of each wave
    __shared__ int s_bad;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int p = blockIdx.x * GP_PLAN_THREADS + t;
    const int64_t e64 = p < P ? sel[p] : -1;
    if (t < E) s_cnt[t] = 0;
    if (t == 0) s_bad = 0;
    for (int i = t; i < GP_PLAN_WAVES * MAX_EXPERTS / 4; i += GP_PLAN_THREADS)
        reinterpret_cast<int*>(&s_wcnt[0][0])[i] = 0;
    const bool ok = e64 >= 0 && e64 < E;
    const int e = ok ? (int)e64 : 0;
    uint64_t eq = __ballot(ok);
#pragma unroll
    for (int b = 0; b < 10; ++b)
    {
        const bool bit = ok && ((e >> b) & 1);
        const uint64_t m = __ballot(bit);
        eq &= bit ? m : ~m;
    }
    const int cin = __popcll(eq & gp_lanes_below(lane));
    const bool lead = ok && cin == 0;   // lowest lane of its expert's group
    __syncthreads();
    if (lead) s_wcnt[wv][e] = (unsigned char)__popcll(eq);
    else if (!ok && e64 != -1) atomicAdd(&s_bad, 1);
    __syncthreads();
    if (ok)
    {
        int r = cin;
        for (int v = 0; v < wv; ++v) r += s_wcnt[v][e];
        g.pick_c[p] = r;
    }
    if (lead) atomicAdd(&s_cnt[e], __popcll(eq));
    __syncthreads();
    int* cc = g.ccnt + (size_t)blockIdx.x * (E + 1);
    if (t < E) cc[t] = s_cnt[t];
    if (t == 0) cc[E] = s_bad;
}

// Inclusive scan over the 64 lanes of a wave.
__device__ __forceinline__ int gp_wave_scan(int v, int lane)
{
#pragma unroll
    for (int d = 1; d < 64; d <<= 1)
    {
        const int o = __shfl_up(v, d);
        if (lane >= d) v += o;
    }
    return v;
}

// Pass 2, one workgroup per chunk: expert e's picks in earlier chunks (base_e) and in all chunks (its slot count),
// slot offsets by a scan of the counts, and the jobs opened before the chunk, sum over e of ceil(base_e / 8) (the
// expert's ranks 0, 8, 16, ... below base_e); a pick's global rank is base_e plus its rank in the chunk, and a pick
// of rank r opens a job when r % 8 == 0, numbered after the chunk's earlier openers. Workgroup 0 also writes the
// counts, offsets, header and the GEMM's expert order.
__global__ __launch_bounds__(GP_PLAN_THREADS) void gp_place_kernel(const int64_t* __restrict__ sel, int P, int E,
                                                                   GPlan g)
{
    __shared__ int s_base[MAX_EXPERTS];
    __shared__ int s_off[MAX_EXPERTS];
    __shared__ __align__(16) int s_nsl[MAX_EXPERTS];
    __shared__ int s_wtot[GP_PLAN_WAVES], s_wjob[GP_PLAN_WAVES], s_wop[GP_PLAN_WAVES];
    __shared__ int s_bad;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int c = blockIdx.x, nch = gridDim.x;
    const int p = c * GP_PLAN_THREADS + t;
    const int64_t e64 = p < P ? sel[p] : -1;
    const bool ok = e64 >= 0 && e64 < E;
    const int e = ok ? (int)e64 : 0;
    const int rc = ok ? g.pick_c[p] : 0;
    if (t == 0) s_bad = 0;
    int base = 0, tot = 0;
    if (t < E)
    {
#pragma unroll 8
        for (int k = 0; k < nch; ++k)
        {
            const int v = g.ccnt[(size_t)k * (E + 1) + t];
            tot += v;
            base += k < c ? v : 0;
        }
    }
    const int inc = gp_wave_scan(tot, lane);
    const int jinc = gp_wave_scan((base + 7) >> 3, lane);
    if (lane == 63)
    {
        s_wtot[wv] = inc;
        s_wjob[wv] = jinc;
    }
    __syncthreads();
    if (c == 0 && t < nch) atomicAdd(&s_bad, g.ccnt[(size_t)t * (E + 1) + E]);
    int pre = 0, jbase = 0;
    for (int v = 0; v < GP_PLAN_WAVES; ++v)
    {
        pre += v < wv ? s_wtot[v] : 0;
        jbase += s_wjob[v];
    }
    const int off_e = pre + inc - tot;
    if (t < E)
    {
        s_base[t] = base;
        s_off[t] = off_e;
        if (c == 0)
        {
            g.cnt[t] = tot;
            g.off[t] = off_e;
            if (t == E - 1)
            {
                g.off[E] = off_e + tot;
                g.hdr[0] = off_e + tot;
            }
        }
    }
    __syncthreads();
    if (c == 0)
    {
        // experts by descending slot count, ties by ascending id: a GEMM workgroup's time grows with its expert's
        // slots (passes, and the blocks of the last pass), so the longest workgroups go first and the short ones
        // fill the end of the launch
        if (t == 0) g.hdr[1] = s_bad;
        s_nsl[t] = t < E ? tot : -1;
        __syncthreads();
        int rk = 0;
        for (int k = 0; k < E; k += 4)   // 16-byte broadcast reads; entries past E are -1
        {
            const int4 pk = *reinterpret_cast<const int4*>(&s_nsl[k]);
            rk += (pk.x > tot || (pk.x == tot && k < t)) + (pk.y > tot || (pk.y == tot && k + 1 < t)) +
                  (pk.z > tot || (pk.z == tot && k + 2 < t)) + (pk.w > tot || (pk.w == tot && k + 3 < t));
        }
        if (t < E) g.eord[rk] = t;
    }
    const int r = ok ? s_base[e] + rc : 0;
    const bool opener = ok && (r & 7) == 0;
    const uint64_t om = __ballot(opener);
    if (lane == 0) s_wop[wv] = __popcll(om);
    __syncthreads();
    int job = jbase + __popcll(om & gp_lanes_below(lane));
    for (int v = 0; v < wv; ++v) job += s_wop[v];
    if (p < P)
    {
        if (ok)
        {
            const int s = s_off[e] + r;
            g.slot_pick[s] = p;
            g.slot_e[s] = e;
            if (opener) g.slot_job[s] = job;
            g.pick_slot[p] = s;
            g.pick_c[p] = r;
        }
        else g.pick_slot[p] = -1;
    }
}

// Pass 3, one thread per token: its picks in (job, pick) order with their fp32 weights. A pick of global rank c
// reads its job number from the slot of its job's opening pick, c % 8 slots before its own.
__global__ __launch_bounds__(GP_ORDER_THREADS) void gp_order_kernel(const void* w, int w_half, int M, int topk, GPlan g)
{
    const int tk = blockIdx.x * GP_ORDER_THREADS + threadIdx.x;
    if (tk >= M) return;
    // loops unrolled to MAX_TOPK with k < topk guards, so the per-pick arrays stay in registers
    int ps[MAX_TOPK], jb[MAX_TOPK];
    int n = 0;
#pragma unroll
    for (int k = 0; k < MAX_TOPK; ++k)
    {
        const int p = tk * topk + k;
        const int s = k < topk ? g.pick_slot[p] : -1;
        ps[k] = s;
        jb[k] = s >= 0 ? g.slot_job[s - (g.pick_c[p] & 7)] : 0;
        n += s >= 0;
    }
    g.tok_npk[tk] = n;
#pragma unroll
    for (int k = 0; k < MAX_TOPK; ++k)
    {
        if (ps[k] < 0) continue;
        int r = 0;
#pragma unroll
        for (int k2 = 0; k2 < MAX_TOPK; ++k2)
            r += ps[k2] >= 0 && (jb[k2] < jb[k] || (jb[k2] == jb[k] && k2 < k));
        const int p = tk * topk + k;
        g.tok_slot[tk * topk + r] = ps[k];
        g.tok_w[tk * topk + r] = w_half ? h2f_bits(reinterpret_cast<const uint16_t*>(w)[p])
                                        : reinterpret_cast<const float*>(w)[p];
    }
}

// ---------------------------------------------------------------------------------------------------------------
// transforms: one wave per slot, or per (token, group of blocks); each 16-lane row of the wave takes one 128-block,
// 8 elements per lane (16-byte loads), 4 blocks per round; exact rounding points
// ---------------------------------------------------------------------------------------------------------------

constexpr int GP_TW = 4;   // waves per transform workgroup
constexpr int GP_TU = 2;   // rounds of 4 blocks per chunk of the input transform (two chunks' loads in flight)
constexpr int GP_TA = 3;   // rounds of 4 blocks per SwiGLU-transform wave (one wave covers I = 1536)

// Elements 8li..8li+7 of 128-block b (one lane of a 16-lane row), rounded to fp16, into the accumulator-chain input
// layout: fp32, position tk * 16 + 4j + q holds row 2q + {0, 1, 8, 9}[j] of tile row tk (the rows chain j of every
// output column reads in tile row tk, in its order)
__device__ __forceinline__ void xg_store_row(float* dst, int b, int li, const float (&v)[8])
{
    float r[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) r[k] = h2f_bits((uint16_t)f2h_bits(v[k]));
    float* d = dst + (size_t)b * 128 + (li >> 1) * 16 + 8 * (li & 1);
    *reinterpret_cast<float4*>(d) = float4{ r[0], r[2], r[4], r[6] };
    *reinterpret_cast<float4*>(d + 4) = float4{ r[1], r[3], r[5], r[7] };
}

// prep_block (ft_core.h:97-102) of the gate and up inputs of slot s (one wave per slot). XL: fp32 in the
// accumulator-chain layout (xg_store_row), else fp16 in the MFMA layout (gp_store_row).
template <bool XL>
__global__ __launch_bounds__(GP_TW * 64) void gp_prep_kernel(const uint64_t* __restrict__ ptrs,
                                                             const uint16_t* __restrict__ x, int H, int topk, int cap,
                                                             GPlan g, void* __restrict__ xt_out)
{
    uint16_t* xt = static_cast<uint16_t*>(xt_out);
    float* xtf = static_cast<float*>(xt_out);
    const int lane = threadIdx.x & 63, rl = lane >> 4, li = lane & 15;
    const int s = blockIdx.x * GP_TW + (threadIdx.x >> 6);
    if (s >= g.hdr[0]) return;
    const int nblk = H / 128;
    const int e = g.slot_e[s], tok = g.slot_pick[s] / topk;
    const gptr<uint16_t> su0 = gaddr<uint16_t>(ptrs[(size_t)e * 9 + 3]);
    const gptr<uint16_t> su1 = gaddr<uint16_t>(ptrs[(size_t)e * 9 + 5]);
    const uint16_t* xr = x + (size_t)tok * H;
    uint16_t* d0 = xt + (size_t)s * H;
    uint16_t* d1 = xt + ((size_t)cap + s) * H;
    float* f0 = xtf + (size_t)s * H;
    float* f1 = xtf + ((size_t)cap + s) * H;
    constexpr int CH = 4 * GP_TU;   // blocks per chunk
    uint4 xv[2][GP_TU], g0[2][GP_TU], g1[2][GP_TU];
    auto load = [&](int buf, int c0) {
#pragma unroll
        for (int k = 0; k < GP_TU; ++k)
        {
            const int o = min(c0 + 4 * k + rl, nblk - 1) * 128 + li * 8;
            xv[buf][k] = *reinterpret_cast<const uint4*>(xr + o);
            g0[buf][k] = gld16(su0, o);
            g1[buf][k] = gld16(su1, o);
        }
    };
    auto work = [&](int buf, int c0) {
#pragma unroll
        for (int k = 0; k < GP_TU; ++k)
        {
            const int b = c0 + 4 * k + rl;
            if constexpr (XL)
            {
                float u[8], v[8];
                prep_block_row_p(u, xv[buf][k], g0[buf][k]);
                prep_block_row_p(v, xv[buf][k], g1[buf][k]);
                if (b < nblk)
                {
                    xg_store_row(f0, b, li, u);
                    xg_store_row(f1, b, li, v);
                }
            }
            else
            {
                uint32_t u[4], v[4];
                prep_block_row_h(u, xv[buf][k], g0[buf][k]);
                prep_block_row_h(v, xv[buf][k], g1[buf][k]);
                if (b < nblk)
                {
                    gp_store_row(d0, b, li, u);
                    gp_store_row(d1, b, li, v);
                }
            }
        }
    };
    // two chunk buffers: the next chunk's loads are in flight while the current one is transformed
    load(0, 0);
    for (int c0 = 0; c0 < nblk; c0 += 2 * CH)
    {
        if (c0 + CH < nblk) load(1, c0 + CH);
        work(0, c0);
        if (c0 + 2 * CH < nblk) load(0, c0 + 2 * CH);
        if (c0 + CH < nblk) work(1, c0 + CH);
    }
}

// fwd_phase phase 1 (ft_core.h:974-991), one wave per (slot, 4 * GP_TA blocks of I): per 128-block, out_block of
// gate and up, r16(act_mul), down prep_block, stored in the GEMM input layout
template <bool XL>
__global__ __launch_bounds__(GP_TW * 64) void gp_act_kernel(const uint64_t* __restrict__ ptrs, int I, int cap, GPlan g,
                                                            const uint16_t* __restrict__ ygu, const float* silu_tab,
                                                            float act_limit, void* __restrict__ xd_out)
{
    uint16_t* xd = static_cast<uint16_t*>(xd_out);
    const int lane = threadIdx.x & 63, rl = lane >> 4, li = lane & 15;
    const int nbi = I / 128, nch = (nbi + 4 * GP_TA - 1) / (4 * GP_TA);
    const int item = blockIdx.x * GP_TW + (threadIdx.x >> 6);
    const int s = item / nch, c0 = (item % nch) * 4 * GP_TA;
    if (s >= g.hdr[0]) return;
    const int e = g.slot_e[s];
    const gptr<uint16_t> svh_g = gaddr<uint16_t>(ptrs[(size_t)e * 9 + 4]);
    const gptr<uint16_t> svh_u = gaddr<uint16_t>(ptrs[(size_t)e * 9 + 6]);
    const gptr<uint16_t> suh_d = gaddr<uint16_t>(ptrs[(size_t)e * 9 + 7]);
    const uint16_t* yg = ygu + (size_t)s * I;
    const uint16_t* yu = ygu + ((size_t)cap + s) * I;
    uint16_t* dst = xd + (size_t)s * I;
    float* dstf = static_cast<float*>(xd_out) + (size_t)s * I;
    // GP_TA rounds of 4 blocks in three phases kept apart by scheduling barriers (left to itself the compiler sinks
    // each round's loads next to their use): all loads; the output transforms and every silu lookup; the
    // activation, input transform and stores
    {
        float gv[GP_TA][8], uv[GP_TA][8], ev[GP_TA][8];
        uint4 gh[GP_TA], uh[GP_TA], sg[GP_TA], su[GP_TA], sd[GP_TA];
#pragma unroll
        for (int k = 0; k < GP_TA; ++k)
        {
            const int o = min(c0 + 4 * k + rl, nbi - 1) * 128 + li * 8;
            gh[k] = *reinterpret_cast<const uint4*>(yg + o);
            uh[k] = *reinterpret_cast<const uint4*>(yu + o);
            sg[k] = gld16(svh_g, o);
            su[k] = gld16(svh_u, o);
            sd[k] = gld16(suh_d, o);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < GP_TA; ++k)
        {
            out_block_row_h(gv[k], gh[k], sg[k]);
            out_block_row_h(uv[k], uh[k], su[k]);
        }
#pragma unroll
        for (int k = 0; k < GP_TA; ++k)
#pragma unroll
            for (int j = 0; j < 8; ++j) ev[k][j] = silu_tab[f2h_bits(gv[k][j]) & 0xFFFFu];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < GP_TA; ++k)
        {
            const int b = c0 + 4 * k + rl;
            float av[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) av[j] = r16(act_mul_s(ev[k][j], uv[k][j], act_limit));
            if constexpr (XL)
            {
                prep_block_row_fp(av, sd[k]);
                if (b < nbi) xg_store_row(dstf, b, li, av);
            }
            else
            {
                uint32_t ah[4];
                prep_block_row_fh(ah, av, sd[k]);
                if (b < nbi) gp_store_row(dst, b, li, ah);
            }
        }
    }
}

// out_block (ft_core.h:1016) of every expert output block and the weighted sum in job order (ft_core.h:1020-1033),
// one wave per (token, group of 4 blocks): each 16-lane row takes one block; lane k < npk holds the token's k-th pick
// (slot, weight, output scales), read back per pick with readlane; four picks' loads are issued before their four
// terms are added in order. Rows of tokens without a valid pick become 0.
constexpr int GP_CK = 4;   // picks whose loads a combine wave keeps in flight

__global__ __launch_bounds__(GP_TW * 64) void gp_comb_kernel(const uint64_t* __restrict__ ptrs, int H, int M, int topk,
                                                             GPlan g, const uint16_t* __restrict__ yraw,
                                                             float* __restrict__ out)
{
    const int lane = threadIdx.x & 63, rl = lane >> 4, li = lane & 15;
    const int nbh = H / 128, ngr = (nbh + 3) / 4;
    const int item = blockIdx.x * GP_TW + (threadIdx.x >> 6);
    const int tok = item / ngr, b = (item % ngr) * 4 + rl;
    if (tok >= M) return;
    const int npk = g.tok_npk[tok];
    int my_s = 0;
    float my_w = 0.f;
    uint64_t my_p = 0;
    if (lane < npk)
    {
        my_s = g.tok_slot[tok * topk + lane];
        my_w = g.tok_w[tok * topk + lane];
        my_p = ptrs[(size_t)g.slot_e[my_s] * 9 + 8];
    }
    const int o = min(b, nbh - 1) * 128 + li * 8;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    for (int k0 = 0; k0 < npk; k0 += GP_CK)
    {
        uint4 yh[GP_CK];
        uint4 sv[GP_CK];
        float wk[GP_CK];
#pragma unroll
        for (int i = 0; i < GP_CK; ++i)
        {
            const int k = min(k0 + i, npk - 1);
            const int s = __builtin_amdgcn_readlane(my_s, k);
            wk[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_w), k));
            const uint64_t pa = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(my_p >> 32), k) << 32) |
                                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)my_p, k);
            yh[i] = *reinterpret_cast<const uint4*>(yraw + (size_t)s * H + o);
            sv[i] = gld16(gaddr<uint16_t>(pa), o);
        }
#pragma unroll
        for (int i = 0; i < GP_CK; ++i)
        {
            if (k0 + i >= npk) break;
            float v[8];
            out_block_row_h(v, yh[i], sv[i]);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = acc[j] + wk[i] * v[j];
        }
    }
    if (b < nbh)
    {
        float* orow = out + (size_t)tok * H + b * 128 + li * 8;
        *reinterpret_cast<float4*>(orow) = float4{ acc[0], acc[1], acc[2], acc[3] };
        *reinterpret_cast<float4*>(orow + 4) = float4{ acc[4], acc[5], acc[6], acc[7] };
    }
}

// ---------------------------------------------------------------------------------------------------------------
// MFMA grouped GEMM: y[slot][n] = sum_k x[slot][k] W_e[k][n] for every slot of every expert
// ---------------------------------------------------------------------------------------------------------------

constexpr int GP_NW = 8;           // waves per GEMM workgroup
constexpr int GP_CPW = 2;          // tile columns per wave (each A fragment read from LDS feeds GP_CPW MFMAs)
constexpr int GP_WCOLS = 16 * GP_NW * GP_CPW;   // output columns per workgroup (256)
constexpr int GP_XPW = GP_MT / GP_NW;           // slots whose input chunk each wave loads per group
constexpr int GP_NG = 2;           // ring depth (groups of 8 tile rows): 2 keeps two workgroups per CU
constexpr int GP_XS = 136;         // fp16 stride of one slot's group chunk in LDS (128 + 8: conflict-free reads)

typedef __attribute__((address_space(3))) void gp_lds_void;

template <int N>
__device__ __forceinline__ void gp_wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without __syncthreads' release fence: that fence waits for vmcnt(0), i.e. for every LDS-direct
// load still in flight, which would drain the prefetch ring at every group. Each wave has already waited for its own
// loads of the group it is about to read; the barrier only has to order those waits (and the previous group's LDS
// reads) across the waves. The "memory" clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void gp_barrier() { asm volatile("s_barrier" ::: "memory"); }

struct GemmArgs
{
    const uint64_t* ptrs;
    int mat_base, nmat;        // first matrix of the launch (0 gate, 1 up, 2 down) and how many
    int kdim, ndim, cap, E;
    GPlan g;
    const uint16_t* xin;       // [mats][cap][kdim] fp16, GEMM input layout
    uint16_t* yout;            // [mats][cap][ndim] fp16: out_block's leading r16 (ft_core.h:109) applied here
};

// Grid: 8 * ceil(E / 8) * (ndim / 256) * matrices, XCD-major. Workgroup = 8 waves x 2 tile columns = 256 output
// columns of one matrix of one expert; the expert's slots go through in passes of GP_MT. Per group of 8 tile rows every
// wave decodes its 16 tiles and, per pair of tile rows, reads one A fragment (16 slots x 32 k) per row block of the
// pass and runs 2 MFMAs (16x16x32) with it, one per column. The tiles stream through per-wave LDS rings and the slots'
// inputs through a shared ring, both filled by LDS-direct loads GP_NG - 1 groups ahead; one workgroup barrier per group
// (group g landed for every wave; every wave is past group g - 1, whose slots are refilled after it).
template <int K>
__global__ __launch_bounds__(GP_NW * 64) void gp_gemm_kernel(GemmArgs a)
{
    constexpr int TB = 32 * K, RB = GP_CPW * TB, GB = 8 * RB, NG = GP_NG;
    constexpr int NLD = GB / 256;                 // trellis dword loads per lane per group
    constexpr int NV = NLD + GP_XPW;              // vector memory instructions per wave per group
    static_assert(GB % 256 == 0, "group of tiles must split into whole wave loads");
    extern __shared__ __align__(16) uint8_t gp_lds[];
    // the wave index in a scalar register, so every LDS-DMA destination (M0) is scalar arithmetic
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    // XCD-aware order: workgroups are dispatched round-robin over the 8 XCDs (XCD = linear id % 8), so every
    // workgroup of the ei-th expert of the dispatch order gets a linear id = ei (mod 8) and the expert's slot inputs
    // are fetched into one L2
    const int nch = a.ndim / GP_WCOLS, per = nch * a.nmat;
    const int xcd = blockIdx.x % 8, j = blockIdx.x / 8;
    const int ei = (j / per) * 8 + xcd, rr0 = j % per;
    if (ei >= a.E) return;
    const int e = a.g.eord[ei];   // experts with the most slots first
    const int nc = rr0 % nch;
    const int mat = a.mat_base + rr0 / nch;
    const int s_begin = a.g.off[e], s_end = a.g.off[e + 1];
    if (s_begin >= s_end) return;
    const int TN = a.ndim / 16, TK = a.kdim / 16, ngroups = TK / 8;
    const int t0 = (nc * GP_NW + wave) * GP_CPW;                     // this wave's first tile column
    uint8_t* ring = gp_lds + wave * NG * GB;                          // [NG][8 tile rows][GP_CPW columns][TB]
    uint16_t* xring = reinterpret_cast<uint16_t*>(gp_lds + GP_NW * NG * GB);   // [NG][64 slots][GP_XS]
    const uint8_t* tr = reinterpret_cast<const uint8_t*>(a.ptrs[(size_t)e * 9 + mat]);
    const size_t gstride = (size_t)TN * TB;                           // bytes per tile row of the matrix
    uint8_t* cb = const_cast<uint8_t*>(uniform_ptr(tr + (size_t)t0 * TB));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(cb, (short)0, (int)((size_t)TK * gstride),
                                                                        0x00020000);
    const int gs = (int)gstride;
    int voff[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i)
    {
        const int byte = i * 256 + lane * 4;   // within the group's [8][GP_CPW][TB] block
        voff[i] = (byte / RB) * gs + (byte % RB);
    }
    const LaneDec d = lane_dec(lane, K);
    const uint16_t* xin = a.xin + (size_t)(mat - a.mat_base) * a.cap * a.kdim;
    // the slots' inputs through a buffer resource too: the lane's 4 bytes as the vector offset, row and group in the
    // scalar offset
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(uniform_ptr(reinterpret_cast<const uint8_t*>(xin))), (short)0,
        (int)((size_t)a.cap * a.kdim * 2), 0x00020000);
    uint16_t* yout = a.yout + (size_t)(mat - a.mat_base) * a.cap * a.ndim;
    const int q = lane >> 4, i16 = lane & 15;

    for (int c0 = s_begin; c0 < s_end; c0 += GP_MT)
    {
        const int T = min(GP_MT, s_end - c0);
        // byte offsets of the input rows this wave loads, the same in every lane (slots past the pass read the pass's
        // last slot): the scalar offset of its LDS-direct loads, whose vector offset is the lane's 4 bytes
        int xrow[GP_XPW];
#pragma unroll
        for (int j = 0; j < GP_XPW; ++j) xrow[j] = (c0 + min(wave * GP_XPW + j, T - 1)) * a.kdim * 2;
        const int xl = lane * 4;
        auto issue = [&](int g) {
            uint8_t* dst = ring + (g % NG) * GB;
#pragma unroll
            for (int i = 0; i < NLD; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (gp_lds_void*)(dst + i * 256), 4, voff[i], g * 8 * gs, 0,
                                                         0);
            uint16_t* xd = xring + (size_t)(g % NG) * GP_MT * GP_XS;
#pragma unroll
            for (int j = 0; j < GP_XPW; ++j)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (gp_lds_void*)(xd + (wave * GP_XPW + j) * GP_XS), 4, xl,
                                                         xrow[j] + g * 256, 0, 0);
        };
        // the pass with its NMB = ceil(T / 16) row blocks of 16 slots: MFMAs and input fragments of empty blocks
        // are not issued
        auto pass = [&](auto nmb_c) {
            constexpr int NMB = decltype(nmb_c)::value;
            float4v acc[GP_CPW][NMB];
#pragma unroll
            for (int c = 0; c < GP_CPW; ++c)
#pragma unroll
                for (int mb = 0; mb < NMB; ++mb) acc[c][mb] = float4v{ 0.f, 0.f, 0.f, 0.f };
            __syncthreads();   // previous pass done with the rings
#pragma unroll
            for (int g = 0; g < NG - 1; ++g)
                if (g < ngroups) issue(g);
            for (int g = 0; g < ngroups; ++g)
            {
                if (g + NG - 2 < ngroups) gp_wait_vmcnt<(NG - 2) * NV>();   // this wave's loads of group g landed
                else gp_wait_vmcnt<0>();
                gp_barrier();   // every wave's loads of group g landed; every wave is done with group g - 1
                if (g + NG - 1 < ngroups) issue(g + NG - 1);   // into the slots of group g - 1
                const uint8_t* sl = ring + (g % NG) * GB;
                const uint16_t* xs = xring + (size_t)(g % NG) * GP_MT * GP_XS;
#pragma unroll
                for (int rp = 0; rp < 4; ++rp)
                {
                    // the trellis words of this pair of tile rows (the next pair's reads go out under this decode)
                    uint32_t wd[GP_CPW][2][2];
#pragma unroll
                    for (int c = 0; c < GP_CPW; ++c)
#pragma unroll
                        for (int h = 0; h < 2; ++h)
                        {
                            const uint8_t* tp = sl + (2 * rp + h) * RB + c * TB;
                            wd[c][h][0] = *reinterpret_cast<const uint32_t*>(tp + d.o0);
                            wd[c][h][1] = *reinterpret_cast<const uint32_t*>(tp + d.o1);
                        }
                    half8 A[NMB];
#pragma unroll
                    for (int mb = 0; mb < NMB; ++mb)
                        A[mb] = *reinterpret_cast<const half8*>(xs + (mb * 16 + i16) * GP_XS + q * 32 + rp * 8);
                    half8 B[GP_CPW];
#pragma unroll
                    for (int c = 0; c < GP_CPW; ++c)
                    {
                        const half4 B0 = decode4<K>(wd[c][0][0], wd[c][0][1], d.sh);
                        const half4 B1 = decode4<K>(wd[c][1][0], wd[c][1][1], d.sh);
                        B[c] = half8{ B0[0], B0[1], B0[2], B0[3], B1[0], B1[1], B1[2], B1[3] };
                    }
                    // raised wave priority while this wave issues its MFMAs: the matrix pipe is refilled as soon as
                    // it frees, and the other waves of the SIMD take the VALU slots in between
                    __builtin_amdgcn_s_setprio(1);
#pragma unroll
                    for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
                        for (int c = 0; c < GP_CPW; ++c)
                            acc[c][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mb], B[c], acc[c][mb], 0, 0, 0);
                    __builtin_amdgcn_s_setprio(0);
                }
            }
            // D[i][n]: lane holds rows 4q + rr of each 16-slot block, column (t0 + c) * 16 + i16
#pragma unroll
            for (int c = 0; c < GP_CPW; ++c)
#pragma unroll
                for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
                    {
                        const int sl = mb * 16 + q * 4 + rr;
                        if (sl < T)
                            yout[(size_t)(c0 + sl) * a.ndim + (t0 + c) * 16 + i16] = (uint16_t)f2h_bits(acc[c][mb][rr]);
                    }
        };
        static_assert(GP_MT == 80, "one case per row-block count");
        switch ((T + 15) / 16)
        {
            case 1: pass(std::integral_constant<int, 1>{}); break;
            case 2: pass(std::integral_constant<int, 2>{}); break;
            case 3: pass(std::integral_constant<int, 3>{}); break;
            case 4: pass(std::integral_constant<int, 4>{}); break;
            default: pass(std::integral_constant<int, 5>{}); break;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// EXACT at prefill sizes: the reference's accumulator chains, each weight decoded once per pass of up to 64 slots
// ---------------------------------------------------------------------------------------------------------------
//
// The reference's EXACT sum (tile_accum<M,EXACT>, ft_core.h:313-345) gives every output column n four fp32
// accumulators; accumulator j takes, in each tile row tk, the products of rows 2q + {0, 1, 8, 9}[j] for q = 0..3, in
// that order, tile rows ascending, and the four are reduced (a0 + a1) + (a2 + a3) (gemv_block, ft_core.h:377-386).
// Here each chain step runs on the matrix cores. v_mfma_f32_16x16x1_4b_f32 computes four independent 16x16 rank-1
// updates D_b = C_b + A_b B_b^T with K = 1. Per element that is one product added to one accumulator, and both
// operands are fp16 values, so the product is exact in fp32 and D = RN(C + A B) = fmaf(A, B, C), the reference's
// chain step. A probe on MI355X matched fmaf bit for bit on 4,096,000 elements (zeros, signed zeros and near-cancelling
// sums included). Block b is chain j = b:
//   - B: lane 16j + n holds chain j's weight of column n at step q. A lane decodes exactly the four weights its chain
//     needs from each tile (stream indices 32 (n % 8) + 4 (n / 8) + j + 8q of the tile's stream, a3/PERM), and each
//     decoded weight serves all the pass's slots.
//   - A: lane 16j + m holds slot m's input for chain j at step q, x[slot][tk * 16 + 2q + off_j] (the input layout of
//     xg_store_row): one ds_read_b128 per lane gives q = 0..3.
//   - D: chain j of (slot 4 (l / 16) + i, column l % 16) sits in register 4j + i of lane l. The reduction
//     (a0 + a1) + (a2 + a3) is then four registers of one lane.
// A wave takes one tile column (16 outputs) with its 4 chains for every slot of the pass, in blocks of 16 slots (one
// MFMA per block and step). Every accumulator is one chain of fused multiply-adds in the reference's order, so the
// results are bit-identical to the decode path's.

// Waves per workgroup: 8 tile columns share one input ring. With the rings (76 KB of LDS at K=3) two workgroups fit
// a CU, 4 waves per SIMD, which needs at most 128 VGPRs. Against 4-wave workgroups at 2 waves per SIMD this measured
// 9.7 against 10.6 ms per config-4 layer.
constexpr int XG_NW = 8;
constexpr int XG_COLS = 16 * XG_NW;         // output columns per workgroup (a tile column per wave)
constexpr int XG_TC = XG_COLS / 16;         // tile columns per workgroup
constexpr int XG_MS = 64;                   // slots per pass
constexpr int XG_NG = 2;                    // ring depth (groups of 8 tile rows)
constexpr int XG_XROW = 8 * 16 * 4;         // input bytes of one slot per group: 8 tile rows x 16 rows x fp32
constexpr int XG_XGB = XG_MS * XG_XROW;     // input bytes per group (32 KB)
// Slots past a pass's whole blocks of 16 run as VALU chains when there are at most XG_REM of them, else as one more
// MFMA block. A VALU chain slot costs a 16-byte LDS read and 4 v_fmac_f32 per tile row against a padded block's 4
// MFMAs; at config 4 (about 57 slots per expert) thresholds 4, 6 and 8 measured 8.61, 8.60 and 8.70 ms per layer
// against 8.95 ms with padding only.
constexpr int XG_REM = 6;
typedef float xg_acc __attribute__((ext_vector_type(16)));   // one 16-slot block of a wave's 4 x 16 x 16 accumulators

struct XgArgs
{
    const uint64_t* ptrs;
    int mat_base, nmat;        // first matrix of the launch (0 gate, 1 up, 2 down) and how many
    int kdim, ndim, cap, E;
    GPlan g;
    const float* xin;          // [mats][cap][kdim] fp32 (fp16-valued), accumulator-chain layout
    uint16_t* yout;            // [mats][cap][ndim] fp16: out_block's leading r16 (ft_core.h:109) applied here
};

// The 16-bit state of stream index t of a tile: the window of bits ending at (t + 1) K of the circular 256K-bit
// stream (state_scalar, ft_core.h:65-73), as a funnel shift of two words (byte offsets o0, o1 in the tile) by sh.
struct StateDec
{
    uint32_t o0, o1, sh;
};
__device__ __forceinline__ StateDec state_dec(int t, int K)
{
    const int e = (t + 1) * K, words = 8 * K;
    const int wa = e >= 33 ? (e - 33) / 32 : -1;   // e - 32 wa in [33, 64]
    StateDec d;
    d.sh = (uint32_t)(64 - (e - 32 * wa));
    d.o0 = (uint32_t)(4 * ((wa + words) % words));
    d.o1 = (uint32_t)(4 * ((wa + 1 + words) % words));
    return d;
}


// Grid: 8 * ceil(E / 8) * (ndim / XG_COLS) * matrices, XCD-major as the MFMA GEMM. Workgroup = XG_NW waves x 16
// columns (a tile column each, all 4 chains) of one matrix of one expert; the expert's slots go through in passes of
// XG_MS. Per group of 8 tile rows the trellis of the XG_TC tile columns and the pass's inputs arrive by LDS-direct
// loads one group ahead (one workgroup barrier per group); at the end of a pass each lane reduces its outputs' 4
// chains.
template <int K>
__global__ __launch_bounds__(XG_NW * 64) __attribute__((amdgpu_waves_per_eu(4))) void xg_gemm_kernel(XgArgs a)
{
    constexpr int TB = 32 * K, RB = XG_TC * TB, GB = 8 * RB, NG = XG_NG;
    constexpr int NLD = GB / 256 / XG_NW;      // trellis dword loads per lane per group (the waves share a group)
    static_assert(GB % (256 * XG_NW) == 0, "a group of tiles splits into whole loads of the waves");
    extern __shared__ __align__(16) uint8_t xg_lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int nch = a.ndim / XG_COLS, per = nch * a.nmat;
    const int xcd = blockIdx.x % 8, jb = blockIdx.x / 8;
    const int ei = (jb / per) * 8 + xcd, rr0 = jb % per;
    if (ei >= a.E) return;
    const int e = a.g.eord[ei];
    const int nc = rr0 % nch;
    const int mat = a.mat_base + rr0 / nch;
    const int s_begin = a.g.off[e], s_end = a.g.off[e + 1];
    if (s_begin >= s_end) return;
    const int TN = a.ndim / 16, TK = a.kdim / 16, ngroups = TK / 8;
    uint8_t* tring = xg_lds;                                   // [NG][8 tile rows][XG_TC tile columns][TB]
    uint8_t* xring = xg_lds + NG * GB;                         // [NG][XG_MS slots][8 tile rows][4 chains][4] fp32
    const uint8_t* tr = reinterpret_cast<const uint8_t*>(a.ptrs[(size_t)e * 9 + mat]);
    const int gs = TN * TB;                                    // bytes per tile row of the matrix
    uint8_t* cb = const_cast<uint8_t*>(uniform_ptr(tr + (size_t)nc * XG_TC * TB));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(cb, (short)0, (int)((size_t)TK * gs),
                                                                        0x00020000);
    int voff[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i)
    {
        const int byte = (wave * NLD + i) * 256 + lane * 4;   // within the group's [8][XG_TC][TB] block
        voff[i] = (byte / RB) * gs + (byte % RB);
    }
    const float* xin = a.xin + (size_t)(mat - a.mat_base) * a.cap * a.kdim;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(uniform_ptr(reinterpret_cast<const uint8_t*>(xin))), (short)0,
        (int)((size_t)a.cap * a.kdim * 4), 0x00020000);
    uint16_t* yout = a.yout + (size_t)(mat - a.mat_base) * a.cap * a.ndim;
    // this lane's chain and column, and the stream windows of the chain's four weights in each tile
    const int j = lane >> 4, tcl = wave, n = lane & 15;
    StateDec sd[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) sd[q] = state_dec(32 * (n & 7) + 4 * (n >> 3) + j + 8 * q, K);
    const int col0 = nc * XG_COLS;

    for (int c0 = s_begin; c0 < s_end; c0 += XG_MS)
    {
        const int T = min(XG_MS, s_end - c0);
        auto issue = [&](int g, int nsl) {
            uint8_t* dst = tring + (g % NG) * GB;
#pragma unroll
            for (int i = 0; i < NLD; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (gp_lds_void*)(dst + (wave * NLD + i) * 256), 4, voff[i],
                                                         g * 8 * gs, 0, 0);
            // this wave's RPW slot rows of the group (rows of slots past the pass repeat its last slot)
            constexpr int RPW = XG_MS / XG_NW;
            uint8_t* xd = xring + (g % NG) * XG_XGB;
            if (wave * RPW < nsl)
            {
#pragma unroll
                for (int r = 0; r < RPW; ++r)
                {
                    const int sl = wave * RPW + r;
                    const int srow = (c0 + min(sl, T - 1)) * a.kdim * 4 + g * XG_XROW;
#pragma unroll
                    for (int h = 0; h < XG_XROW / 256; ++h)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (gp_lds_void*)(xd + sl * XG_XROW + h * 256), 4,
                                                                 h * 256 + lane * 4, srow, 0, 0);
                }
            }
        };
        // NSL slots in blocks of 16 on the matrix cores, then R <= XG_REM slots past them as VALU chains: lane
        // (j, n) runs slot m's chain j of column n as v_fmac_f32 steps, fmaf(x, w, acc) as each K=1 MFMA step is, in
        // the same step order, on the weights the lane decoded for the MFMAs
        auto pass = [&](auto nsl_c, int R) {
            constexpr int NSL = decltype(nsl_c)::value, NB = NSL / 16;
            xg_acc acc[NB > 0 ? NB : 1];
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[b][r] = 0.f;
            float racc[XG_REM];
#pragma unroll
            for (int m = 0; m < XG_REM; ++m) racc[m] = 0.f;
            __syncthreads();   // the previous pass is done with the rings
            issue(0, NSL + R);
            for (int g = 0; g < ngroups; ++g)
            {
                gp_wait_vmcnt<0>();
                gp_barrier();   // group g landed for every wave; every wave is done with group g - 1
                if (g + 1 < ngroups) issue(g + 1, NSL + R);
                const uint8_t* tl = tring + (g % NG) * GB + tcl * TB;
                // lane (j, m) reads slot 16 b + m's inputs of chain j
                const uint8_t* xl = xring + (g % NG) * XG_XGB + n * XG_XROW + j * 16;
                // lane (j, n) reads remainder slot NSL + m's inputs of chain j (the same 16 bytes for all n)
                const uint8_t* xr = xring + (g % NG) * XG_XGB + NSL * XG_XROW + j * 16;
#pragma unroll
                for (int t8 = 0; t8 < 8; ++t8)
                {
                    const uint8_t* tp = tl + t8 * RB;
                    uint32_t st[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                    {
                        const uint32_t hi = *reinterpret_cast<const uint32_t*>(tp + sd[q].o0);
                        const uint32_t lo = *reinterpret_cast<const uint32_t*>(tp + sd[q].o1);
                        st[q] = __builtin_amdgcn_alignbit(hi, lo, sd[q].sh) & 0xFFFFu;
                    }
                    const half4 wh = codebook4(st[0], st[1], st[2], st[3]);
                    const float w[4] = { (float)wh[0], (float)wh[1], (float)wh[2], (float)wh[3] };
                    float4 xv[NB > 0 ? NB : 1];
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        xv[b] = *reinterpret_cast<const float4*>(xl + b * 16 * XG_XROW + t8 * 64);
                    // steps q = 0..3 of the tile row; the blocks' chains are independent between dependent steps
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        acc[b] = __builtin_amdgcn_mfma_f32_16x16x1f32(xv[b].x, w[0], acc[b], 0, 0, 0);
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        acc[b] = __builtin_amdgcn_mfma_f32_16x16x1f32(xv[b].y, w[1], acc[b], 0, 0, 0);
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        acc[b] = __builtin_amdgcn_mfma_f32_16x16x1f32(xv[b].z, w[2], acc[b], 0, 0, 0);
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        acc[b] = __builtin_amdgcn_mfma_f32_16x16x1f32(xv[b].w, w[3], acc[b], 0, 0, 0);
                    if (R > 0)
                    {
#pragma unroll
                        for (int m = 0; m < XG_REM; ++m)
                            if (m < R)
                            {
                                const float4 x4 = *reinterpret_cast<const float4*>(xr + m * XG_XROW + t8 * 64);
                                racc[m] = __builtin_fmaf(x4.x, w[0], racc[m]);
                                racc[m] = __builtin_fmaf(x4.y, w[1], racc[m]);
                                racc[m] = __builtin_fmaf(x4.z, w[2], racc[m]);
                                racc[m] = __builtin_fmaf(x4.w, w[3], racc[m]);
                            }
                    }
                }
            }
            // chain c of (slot 16 b + 4 (lane / 16) + i, column lane % 16) is register 4c + i of acc[b]: the
            // reference's (a0 + a1) + (a2 + a3), rounded to fp16 (out_block's leading r16)
            const int col = col0 + tcl * 16 + n;
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    const int s = 16 * b + 4 * j + i;
                    const float y = (acc[b][i] + acc[b][4 + i]) + (acc[b][8 + i] + acc[b][12 + i]);
                    if (s < T) yout[(size_t)(c0 + s) * a.ndim + col] = (uint16_t)f2h_bits(y);
                }
            // remainder slots: chain j of (slot, column n) is racc in lane 16 j + n
            if (R > 0)
            {
#pragma unroll
                for (int m = 0; m < XG_REM; ++m)
                    if (m < R)
                    {
                        const float a1 = __shfl(racc[m], n + 16), a2 = __shfl(racc[m], n + 32),
                                    a3 = __shfl(racc[m], n + 48);
                        const float y = (racc[m] + a1) + (a2 + a3);
                        if (j == 0) yout[(size_t)(c0 + NSL + m) * a.ndim + col] = (uint16_t)f2h_bits(y);
                    }
            }
        };
        // slots past the last whole block of 16: up to XG_REM of them as VALU chains, more as one more MFMA block
        const int R = T % 16 <= XG_REM ? T % 16 : 0;
        switch ((T - R + 15) / 16)
        {
            case 0: pass(std::integral_constant<int, 0>{}, R); break;
            case 1: pass(std::integral_constant<int, 16>{}, R); break;
            case 2: pass(std::integral_constant<int, 32>{}, R); break;
            case 3: pass(std::integral_constant<int, 48>{}, R); break;
            default: pass(std::integral_constant<int, 64>{}, 0); break;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------------------------------

template <int K>
static size_t gp_gemm_lds()
{
    return (size_t)GP_NW * GP_NG * 8 * GP_CPW * 32 * K + (size_t)GP_NG * GP_MT * GP_XS * 2;
}

template <int K>
static int gp_gemm_launch(const GemmArgs& a, int nmat, hipStream_t st)
{
    const size_t lds = gp_gemm_lds<K>();
    // opened to what the kernel needs once per process (thread-safe static initialisation)
    static const bool opened = hipFuncSetAttribute(reinterpret_cast<const void*>(gp_gemm_kernel<K>),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess;
    if (!opened) return -1;
    GemmArgs b = a;
    b.nmat = nmat;
    const unsigned grid = (unsigned)(((a.E + 7) / 8) * 8 * (a.ndim / GP_WCOLS) * nmat);
    hipLaunchKernelGGL(gp_gemm_kernel<K>, dim3(grid), dim3(GP_NW * 64), lds, st, b);
    return 0;
}

static int gp_gemm(int K, const GemmArgs& a, int nmat, hipStream_t st)
{
    switch (K)
    {
        case 2: return gp_gemm_launch<2>(a, nmat, st);
        case 3: return gp_gemm_launch<3>(a, nmat, st);
        case 4: return gp_gemm_launch<4>(a, nmat, st);
        case 5: return gp_gemm_launch<5>(a, nmat, st);
        default: return -1;
    }
}

template <int K>
static size_t xg_gemm_lds()
{
    return (size_t)XG_NG * 8 * XG_TC * 32 * K + (size_t)XG_NG * XG_XGB;
}

template <int K>
static int xg_gemm_launch(const XgArgs& a, int nmat, hipStream_t st)
{
    const size_t lds = xg_gemm_lds<K>();
    static const bool opened = hipFuncSetAttribute(reinterpret_cast<const void*>(xg_gemm_kernel<K>),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess;
    if (!opened) return -1;
    XgArgs b = a;
    b.nmat = nmat;
    const unsigned grid = (unsigned)(((a.E + 7) / 8) * 8 * (a.ndim / XG_COLS) * nmat);
    hipLaunchKernelGGL(xg_gemm_kernel<K>, dim3(grid), dim3(XG_NW * 64), lds, st, b);
    return 0;
}

static int xg_gemm(int K, const XgArgs& a, int nmat, hipStream_t st)
{
    switch (K)
    {
        case 2: return xg_gemm_launch<2>(a, nmat, st);
        case 3: return xg_gemm_launch<3>(a, nmat, st);
        case 4: return xg_gemm_launch<4>(a, nmat, st);
        case 5: return xg_gemm_launch<5>(a, nmat, st);
        default: return -1;
    }
}

void launch_grouped_plan(const int64_t* sel, const void* w, int w_half, int P, int topk, int E, const GPlan& g,
                         hipStream_t st)
{
    const int M = P / topk;
    const unsigned nch = (unsigned)((P + GP_PLAN_CHUNK - 1) / GP_PLAN_CHUNK);
    hipLaunchKernelGGL(gp_rank_kernel, dim3(nch), dim3(GP_PLAN_THREADS), 0, st, sel, P, E, g);
    hipLaunchKernelGGL(gp_place_kernel, dim3(nch), dim3(GP_PLAN_THREADS), 0, st, sel, P, E, g);
    hipLaunchKernelGGL(gp_order_kernel, dim3((unsigned)((M + GP_ORDER_THREADS - 1) / GP_ORDER_THREADS)),
                       dim3(GP_ORDER_THREADS), 0, st, w, w_half, M, topk, g);
}

int launch_grouped(const uint64_t* ptrs, const int64_t* sel, const void* w, int w_half, int P, int topk, int E, int H,
                   int I, int Kg, int Ku, int Kd, const uint16_t* x, const GPlan& g, int cap, uint16_t* xt,
                   uint16_t* ygu, uint16_t* xd, uint16_t* yraw, const float* silu_tab, float act_limit, float* out,
                   hipStream_t st)
{
    const int M = P / topk;
    launch_grouped_plan(sel, w, w_half, P, topk, E, g, st);
    const unsigned slot_wgs = (unsigned)((P + GP_TW - 1) / GP_TW);
    hipLaunchKernelGGL(gp_prep_kernel<false>, dim3(slot_wgs), dim3(GP_TW * 64), 0, st, ptrs, x, H, topk, cap, g,
                       static_cast<void*>(xt));
    GemmArgs a;
    a.ptrs = ptrs; a.kdim = H; a.ndim = I; a.cap = cap; a.E = E; a.g = g; a.xin = xt; a.yout = ygu;
    if (Kg == Ku)
    {
        a.mat_base = 0;
        if (gp_gemm(Kg, a, 2, st)) return -1;
    }
    else
    {
        a.mat_base = 0;
        if (gp_gemm(Kg, a, 1, st)) return -1;
        GemmArgs b = a;
        b.mat_base = 1;
        b.xin = xt + (size_t)cap * H;
        b.yout = ygu + (size_t)cap * I;
        if (gp_gemm(Ku, b, 1, st)) return -1;
    }
    const long act_items = (long)P * ((I / 128 + 4 * GP_TA - 1) / (4 * GP_TA));
    hipLaunchKernelGGL(gp_act_kernel<false>, dim3((unsigned)((act_items + GP_TW - 1) / GP_TW)), dim3(GP_TW * 64), 0,
                       st, ptrs, I, cap, g, ygu, silu_tab, act_limit, static_cast<void*>(xd));
    GemmArgs c = a;
    c.mat_base = 2; c.kdim = I; c.ndim = H; c.xin = xd; c.yout = yraw;
    if (gp_gemm(Kd, c, 1, st)) return -1;
    {
        const long items = (long)M * ((H / 128 + 3) / 4);
        hipLaunchKernelGGL(gp_comb_kernel, dim3((unsigned)((items + GP_TW - 1) / GP_TW)), dim3(GP_TW * 64), 0, st, ptrs,
                           H, M, topk, g, yraw, out);
    }
    return 0;
}

int launch_exact_chains(const uint64_t* ptrs, const int64_t* sel, const void* w, int w_half, int P, int topk, int E,
                        int H, int I, int Kg, int Ku, int Kd, const uint16_t* x, const GPlan& g, int cap, float* xt,
                        uint16_t* ygu, float* xd, uint16_t* yraw, const float* silu_tab, float act_limit, float* out,
                        hipStream_t st)
{
    // the chain GEMM addresses its fp32 inputs with 32-bit byte offsets
    if ((size_t)cap * (size_t)(H > I ? H : I) * 4 > (size_t)0x7fffffff) return -1;
    const int M = P / topk;
    launch_grouped_plan(sel, w, w_half, P, topk, E, g, st);
    const unsigned slot_wgs = (unsigned)((P + GP_TW - 1) / GP_TW);
    hipLaunchKernelGGL(gp_prep_kernel<true>, dim3(slot_wgs), dim3(GP_TW * 64), 0, st, ptrs, x, H, topk, cap, g,
                       static_cast<void*>(xt));
    XgArgs a;
    a.ptrs = ptrs; a.kdim = H; a.ndim = I; a.cap = cap; a.E = E; a.g = g; a.xin = xt; a.yout = ygu;
    if (Kg == Ku)
    {
        a.mat_base = 0;
        if (xg_gemm(Kg, a, 2, st)) return -1;
    }
    else
    {
        a.mat_base = 0;
        if (xg_gemm(Kg, a, 1, st)) return -1;
        XgArgs b = a;
        b.mat_base = 1;
        b.xin = xt + (size_t)cap * H;
        b.yout = ygu + (size_t)cap * I;
        if (xg_gemm(Ku, b, 1, st)) return -1;
    }
    const long act_items = (long)P * ((I / 128 + 4 * GP_TA - 1) / (4 * GP_TA));
    hipLaunchKernelGGL(gp_act_kernel<true>, dim3((unsigned)((act_items + GP_TW - 1) / GP_TW)), dim3(GP_TW * 64), 0,
                       st, ptrs, I, cap, g, ygu, silu_tab, act_limit, static_cast<void*>(xd));
    XgArgs c = a;
    c.mat_base = 2; c.kdim = I; c.ndim = H; c.xin = xd; c.yout = yraw;
    if (xg_gemm(Kd, c, 1, st)) return -1;
    {
        const long items = (long)M * ((H / 128 + 3) / 4);
        hipLaunchKernelGGL(gp_comb_kernel, dim3((unsigned)((items + GP_TW - 1) / GP_TW)), dim3(GP_TW * 64), 0, st, ptrs,
                           H, M, topk, g, yraw, out);
    }
    return 0;
}

size_t grouped_gemm_lds_bytes(int K)
{
    switch (K)
    {
        case 2: return gp_gemm_lds<2>();
        case 3: return gp_gemm_lds<3>();
        case 4: return gp_gemm_lds<4>();
        case 5: return gp_gemm_lds<5>();
        default: return 0;
    }
}

}  // namespace gfl
