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
__global__ __launch_bounds__(256) void plan_kernel(const int64_t* __restrict__ sel, const void* __restrict__ w,
                                                   int w_half, int P, int topk, int E, PlanView pv)
{
    __shared__ int s_e[MAX_PICKS], s_c[MAX_PICKS], s_first[MAX_PICKS], s_crank[MAX_PICKS];
    __shared__ int firstpick[MAX_EXPERTS], ucnt[MAX_PICKS], uoff[MAX_PICKS + 1];
    __shared__ int s_U, s_bad, s_job[MAX_PICKS], s_slot[MAX_PICKS];
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
        s_job[p] = s_crank[creator];
        s_slot[p] = slot;
    }
    __syncthreads();
    // per token: its picks in (job, pick) order -> the order of the weighted sum (ft_core.h:1020-1033)
    for (int t0 = t; t0 * topk < P; t0 += blockDim.x)
    {
        int ord[MAX_TOPK];
        int cnt = 0;
        for (int k = 0; k < topk; ++k)
        {
            const int p = t0 * topk + k;
            if (s_e[p] < 0) continue;
            int b = cnt++;
            while (b > 0 && s_job[ord[b - 1]] > s_job[p]) { ord[b] = ord[b - 1]; --b; }
            ord[b] = p;
        }
        for (int k = 0; k < topk; ++k)
        {
            const int p = k < cnt ? ord[k] : -1;
            pv.tok_slot[t0 * topk + k] = p >= 0 ? s_slot[p] : -1;
            pv.tok_w[t0 * topk + k] = p < 0 ? 0.f
                                   : (w_half ? h2f_bits(reinterpret_cast<const uint16_t*>(w)[p])
                                             : reinterpret_cast<const float*>(w)[p]);
        }
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

// One workgroup = NW waves = NW adjacent tile columns (16*NW outputs) of one matrix of one routed expert, all tile
// rows, for up to NS of the expert's slots at a time. Each wave owns one tile column; lane (j = l/16, n = l%16)
// carries the reference's accumulator j of output column n for every slot.
// Trellis bytes are streamed in batches of BR tile rows: each thread issues coalesced 16-byte loads into a ring of
// NRING register batches (so NRING batches are in flight), the batch is written to one of two LDS buffers and the
// waves decode their tile column from there.
//   PREP = true : gate/up; the WG builds xt = prep_block(x_token, suh) for its slots in LDS
//   PREP = false: down; xt (already transformed and permuted) is copied from xin
//   OUTB = true : apply out_block (ft_core.h:1016) to each 128-output block and write final expert outputs
//                 (needs NW = 8)
constexpr int BR = 16;      // tile rows per batch

// Workgroup barrier that only orders LDS traffic: wait for this wave's LDS operations, then s_barrier. Unlike
// __syncthreads it carries no release fence, so outstanding global loads of the prefetch ring stay in flight.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 16-byte load through the global address space (pointers taken from the layer table are generic; a flat load
// would also count against lgkmcnt and be drained by every LDS wait)
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 gload16(const uint8_t* p)
{
    typedef const __attribute__((address_space(1))) u32x4 gu32x4;
    return *(gu32x4*)(p);
}
constexpr int NRING = 4;    // batches in flight per workgroup

template <int K, int NW>
struct Stage
{
    static constexpr int TB = 32 * K;                   // bytes per tile
    static constexpr int RB = NW * TB;                  // bytes per tile-row slice of the workgroup
    static constexpr int BB = BR * RB;                  // bytes per batch
    static constexpr int NCH = BB / 16;                 // 16-byte chunks per batch
    static constexpr int CPT = (NCH + NW * 64 - 1) / (NW * 64);   // chunks per thread
    static constexpr int BBP = CPT * NW * 64 * 16;      // staged bytes per batch incl. the pad the surplus chunks fill
};

template <int K, int NS, bool PREP, int NW, bool OUTB>
__global__ __launch_bounds__(NW * 64) void chain_gemv_kernel(const uint64_t* __restrict__ ptrs, int mat_base,
                                                             int kdim, int ndim, PlanView pv, int topk,
                                                             const uint16_t* __restrict__ xin,
                                                             float* __restrict__ yout)
{
    using St = Stage<K, NW>;
    extern __shared__ __align__(16) uint8_t lds_raw[];
    uint8_t* stage_buf = lds_raw;                                     // [2][BBP]
    uint16_t* lds_x = reinterpret_cast<uint16_t*>(lds_raw + 2 * St::BBP);  // [NS][kdim] fp16, permuted [tk][j][q]
    float* lds_y = reinterpret_cast<float*>(lds_raw + 2 * St::BBP + (size_t)NS * kdim * 2);  // [NS][128] (OUTB)
    const int TN = ndim / 16, TK = kdim / 16, ncb = TN / NW;
    const int u = blockIdx.x / ncb, cb = blockIdx.x % ncb;
    if (u >= pv.hdr[0]) return;
    const int mat = mat_base + blockIdx.y;                 // 0 gate, 1 up, 2 down
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e = pv.uexp[u];
    const uint8_t* tr = reinterpret_cast<const uint8_t*>(ptrs[(size_t)e * 9 + mat]);
    const uint16_t* suh = reinterpret_cast<const uint16_t*>(ptrs[(size_t)e * 9 + 3 + 2 * mat]);
    const uint16_t* svh = reinterpret_cast<const uint16_t*>(ptrs[(size_t)e * 9 + 4 + 2 * mat]);
    const int s_begin = pv.uoff[u], s_end = pv.uoff[u + 1];
    const LaneDec d = lane_dec(lane, K);
    const int j = lane >> 4, n = lane & 15;
    half4 Pm;
#pragma unroll
    for (int r = 0; r < 4; ++r) Pm[r] = (_Float16)((j == (n & 3) && r == (n >> 2)) ? 1.0f : 0.0f);
    const float4v zero = { 0.f, 0.f, 0.f, 0.f };
    const size_t gstride = (size_t)TN * St::TB;            // global bytes between tile rows
    const uint8_t* gbase = tr + (size_t)cb * St::RB;        // tile row 0 of this workgroup's slice
    const int nb = (TK + BR - 1) / BR;
    float* ybase = yout + (size_t)blockIdx.y * (size_t)pv.cap_slots * ndim;

    // chunk c of batch b: tile row b*BR + c/(RB/16), byte (c % (RB/16))*16 of the slice; batches past the end reload
    // the last tile row (in bounds, never consumed) so the ring has no branches
    // every thread moves exactly CPT chunks; chunks past NCH reload chunk c - NCH into the pad (no branches)
#define GFL_LOAD_BATCH(BI, REG)                                                                                  \
    _Pragma("unroll") for (int i_ = 0; i_ < St::CPT; ++i_)                                                       \
    {                                                                                                            \
        const int cr_ = threadIdx.x + i_ * NW * 64;                                                              \
        const int c_ = cr_ < St::NCH ? cr_ : cr_ - St::NCH;                                                      \
        const int row_ = min((BI) * BR + c_ / (St::RB / 16), TK - 1);                                            \
        REG[i_] = gload16(gbase + (size_t)row_ * gstride + (c_ % (St::RB / 16)) * 16);                           \
    }
#define GFL_STORE_BATCH(BUF, REG)                                                                                \
    _Pragma("unroll") for (int i_ = 0; i_ < St::CPT; ++i_)                                                       \
        reinterpret_cast<u32x4*>(stage_buf + (BUF) * St::BBP)[threadIdx.x + i_ * NW * 64] = REG[i_];
    // one pipeline step: publish batch BI from its ring slot, refill the slot with batch BI + 4, decode batch BI
#define GFL_STEP(BI, REG)                                                                                        \
    {                                                                                                            \
        const int b_ = (BI);                                                                                     \
        GFL_STORE_BATCH(b_ & 1, REG)                                                                             \
        lds_barrier();                                                                                           \
        GFL_LOAD_BATCH(b_ + 4, REG)                                                                              \
        const uint8_t* sb_ = wl + (b_ & 1) * St::BBP;                                                            \
        if (b_ < nb)                                                                                             \
        {                                                                                                        \
            _Pragma("unroll") for (int g_ = 0; g_ < BR; g_ += 4)                                                 \
            {                                                                                                    \
                /* four independent tiles: LDS words, decode and MFMA transposition first, then the chains */   \
                uint32_t hi_[4], lo_[4];                                                                         \
                _Pragma("unroll") for (int r_ = 0; r_ < 4; ++r_)                                                 \
                {                                                                                                \
                    hi_[r_] = *reinterpret_cast<const uint32_t*>(sb_ + (g_ + r_) * St::RB + d.o0);              \
                    lo_[r_] = *reinterpret_cast<const uint32_t*>(sb_ + (g_ + r_) * St::RB + d.o1);              \
                }                                                                                                \
                float4v cw_[4];                                                                                  \
                _Pragma("unroll") for (int r_ = 0; r_ < 4; ++r_)                                                 \
                    cw_[r_] = __builtin_amdgcn_mfma_f32_16x16x16f16(Pm, decode4<K>(hi_[r_], lo_[r_], d.sh), zero, \
                                                                    0, 0, 0);                                    \
                _Pragma("unroll") for (int s_ = 0; s_ < NS; ++s_)                                                \
                {                                                                                                \
                    if (s_ < ns)                                                                                 \
                    {                                                                                            \
                        float a_ = acc[s_];                                                                      \
                        _Pragma("unroll") for (int r_ = 0; r_ < 4; ++r_)                                         \
                        {                                                                                        \
                            const int tk_ = b_ * BR + g_ + r_;                                                   \
                            const half4 xv_ = *reinterpret_cast<const half4*>(xl + ((size_t)s_ * TK + tk_) * 16); \
                            a_ = __builtin_fmaf(cw_[r_][0], (float)xv_[0], a_);                                  \
                            a_ = __builtin_fmaf(cw_[r_][1], (float)xv_[1], a_);                                  \
                            a_ = __builtin_fmaf(cw_[r_][2], (float)xv_[2], a_);                                  \
                            a_ = __builtin_fmaf(cw_[r_][3], (float)xv_[3], a_);                                  \
                        }                                                                                        \
                        acc[s_] = a_;                                                                            \
                    }                                                                                            \
                }                                                                                                \
            }                                                                                                    \
        }                                                                                                        \
    }

    for (int c0 = s_begin; c0 < s_end; c0 += NS)
    {
        const int ns = min(NS, s_end - c0);
        // prefetch ring: four named register batches in flight
        u32x4 ring0[St::CPT], ring1[St::CPT], ring2[St::CPT], ring3[St::CPT];
        static_assert(NRING == 4, "ring of four batches");
        GFL_LOAD_BATCH(0, ring0)
        GFL_LOAD_BATCH(1, ring1)
        GFL_LOAD_BATCH(2, ring2)
        GFL_LOAD_BATCH(3, ring3)
        lds_barrier();   // previous pass done with lds_x / lds_y
        if (PREP)
        {
            const int nblk = kdim / 128;
            for (int it = wave; it < ns * nblk; it += NW)
            {
                const int s = it / nblk, b = it % nblk;
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

        float acc[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) acc[s] = 0.f;
        const uint8_t* wl = stage_buf + wave * St::TB;      // this wave's tile inside a staged row slice
        const uint16_t* xl = lds_x + j * 4;
        for (int b0 = 0; b0 < nb; b0 += NRING)
        {
            GFL_STEP(b0, ring0)
            GFL_STEP(b0 + 1, ring1)
            GFL_STEP(b0 + 2, ring2)
            GFL_STEP(b0 + 3, ring3)
        }
#undef GFL_STEP
#undef GFL_STORE_BATCH
#undef GFL_LOAD_BATCH
        const int t = cb * NW + wave;                          // this wave's tile column
#pragma unroll
        for (int s = 0; s < NS; ++s)
        {
            const float a1 = __shfl(acc[s], n + 16), a2 = __shfl(acc[s], n + 32), a3 = __shfl(acc[s], n + 48);
            const float y = (acc[s] + a1) + (a2 + a3);
            if (s < ns && lane < 16)
            {
                if (OUTB) lds_y[s * 128 + wave * 16 + n] = y;
                else ybase[(size_t)(c0 + s) * ndim + t * 16 + n] = y;
            }
        }
        if (OUTB)
        {
            __syncthreads();
            const int blk = cb;                                // NW == 8: one 128-output block per workgroup
            for (int s = wave; s < ns; s += NW)
            {
                float v0 = lds_y[s * 128 + lane], v1 = lds_y[s * 128 + lane + 64];
                out_block_wave(v0, v1, h2f_bits(svh[blk * 128 + lane]), h2f_bits(svh[blk * 128 + lane + 64]));
                ybase[(size_t)(c0 + s) * ndim + blk * 128 + lane] = v0;
                ybase[(size_t)(c0 + s) * ndim + blk * 128 + lane + 64] = v1;
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// gate|up -> out_block -> act -> down-input prep (fwd_phase phase 1, ft_core.h:974-991)
// ---------------------------------------------------------------------------------------------------------------

__global__ __launch_bounds__(256) void act_kernel(const uint64_t* __restrict__ ptrs, PlanView pv,
                                                  const float* __restrict__ ygu, uint16_t* __restrict__ xtd, int I,
                                                  float limit, const float* __restrict__ exp_tab)
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
    float a0 = r16(act_mul(g0, u0, limit, exp_tab)), a1 = r16(act_mul(g1, u1, limit, exp_tab));
    prep_block_wave(a0, a1, h2f_bits(suh_d[ib * 128 + lane]), h2f_bits(suh_d[ib * 128 + lane + 64]));
    uint16_t* dst = xtd + (size_t)s * I;
    dst[perm_pos(ib, lane)] = (uint16_t)f2h_bits(a0);
    dst[perm_pos(ib, lane + 64)] = (uint16_t)f2h_bits(a1);
}

// ---------------------------------------------------------------------------------------------------------------
// down out_block + weighted sum in job order (fwd_phase phases 2-3, ft_core.h:1014-1033)
// ---------------------------------------------------------------------------------------------------------------

__global__ __launch_bounds__(256) void final_kernel(PlanView pv, int M, int topk, const float* __restrict__ yd,
                                                    float* __restrict__ out, int H)
{
    // one thread per output element: o = 0, then += w * y over the token's picks in (job, pick) order
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= M * H) return;
    const int tkn = idx / H, col = idx % H;
    float o = 0.f;
    for (int k = 0; k < topk; ++k)
    {
        const int s = pv.tok_slot[tkn * topk + k];
        if (s < 0) break;
        o = o + pv.tok_w[tkn * topk + k] * yd[(size_t)s * H + col];
    }
    out[idx] = o;
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

void launch_plan(const int64_t* sel, const void* w, int w_half, int P, int topk, int E, const PlanView& pv,
                 hipStream_t st)
{
    hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(256), 0, st, sel, w, w_half, P, topk, E, pv);
}

template <int K, int NS, bool PREP, int NW, bool OUTB>
static void chain_launch(const uint64_t* ptrs, int mat_base, int nmat, int kdim, int ndim, const PlanView& pv,
                         int topk, int umax, const uint16_t* xin, float* yout, hipStream_t st)
{
    const int ncb = ndim / (16 * NW);
    const size_t lds = 2 * (size_t)Stage<K, NW>::BBP + (size_t)NS * kdim * 2 + (OUTB ? (size_t)NS * 128 * 4 : 0);
    auto kern = chain_gemv_kernel<K, NS, PREP, NW, OUTB>;
    static int lds_set = 0;   // largest dynamic LDS this instantiation has been opened up to
    if ((int)lds > lds_set)
    {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)lds);
        lds_set = (int)lds;
    }
    hipLaunchKernelGGL(kern, dim3(umax * ncb, nmat), dim3(NW * 64), lds, st, ptrs, mat_base, kdim, ndim, pv, topk,
                       xin, yout);
}

template <int K, bool PREP>
static void chain_ns(int ns, const uint64_t* ptrs, int mat_base, int nmat, int kdim, int ndim, const PlanView& pv,
                     int topk, int umax, const uint16_t* xin, float* yout, hipStream_t st)
{
    // gate/up: 4 waves (64 outputs) per workgroup; down: 8 waves = one 128-output block, out_block fused
    constexpr int NW = PREP ? 4 : 8;
    constexpr bool OUTB = !PREP;
    if (ns <= 1) chain_launch<K, 1, PREP, NW, OUTB>(ptrs, mat_base, nmat, kdim, ndim, pv, topk, umax, xin, yout, st);
    else if (ns <= 2) chain_launch<K, 2, PREP, NW, OUTB>(ptrs, mat_base, nmat, kdim, ndim, pv, topk, umax, xin, yout, st);
    else if (ns <= 4) chain_launch<K, 4, PREP, NW, OUTB>(ptrs, mat_base, nmat, kdim, ndim, pv, topk, umax, xin, yout, st);
    else chain_launch<K, 8, PREP, NW, OUTB>(ptrs, mat_base, nmat, kdim, ndim, pv, topk, umax, xin, yout, st);
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
                float limit, const float* exp_tab, hipStream_t st)
{
    const int items = smax * (I / 128);
    hipLaunchKernelGGL(act_kernel, dim3((items + 3) / 4), dim3(256), 0, st, ptrs, pv, ygu, xtd, I, limit,
                       exp_tab);
}

void launch_final(const uint64_t* ptrs, const PlanView& pv, const void* w, int w_half, int M, int topk,
                  const float* yd, float* out, int H, hipStream_t st)
{
    const int n = M * H;
    hipLaunchKernelGGL(final_kernel, dim3((n + 255) / 256), dim3(256), 0, st, pv, M, topk, yd, out, H);
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
