// Routed-MoE decode path on gfx950 in two launches: gate|up (with the routing plan and the SwiGLU stage fused in)
// and down (with the output transform and the weighted combine fused in).
//
// Numerics follow the reference's EXACT mode (kernels/cpu_avx2/ft_core.h:313-387, 933-1033) operation for
// operation, so outputs are bit-identical to it:
//   * each output column keeps the reference's four fp32 accumulators (AVX lanes j of tile_accum), each a chain of
//     fused multiply-adds over tile rows, and inside a tile row over the four stream groups q;
//   * the column result is (a0 + a1) + (a2 + a3);
//   * Hadamard/rounding points are those of prep_block / out_block / act_mul;
//   * the weighted sum runs over each token's picks in the reference's job order.
// The chain needs the weights of one (column, accumulator) in q order, while the trellis decodes four consecutive
// stream indices per lane (fixed q, accumulators 0..3). One MFMA 16x16x16 against a constant 0/1 permutation
// matrix moves the decoded tile from the first layout to the second as exact fp32 values.
//
// Cross-workgroup steps use "last one finishes" counters instead of extra launches: a workgroup publishes its
// outputs, then bumps a device-scope acquire-release counter; the one that completes the count runs the dependent
// step (SwiGLU of a 128-block once gate and up of that block are in; the combine of a token's 128-block once all its
// experts' down outputs are in) and re-arms the counter to zero for the next call. Nothing waits on anything.
#include "gfl_device.hpp"
#include "gfl_internal.hpp"

namespace gfl {

// ---------------------------------------------------------------------------------------------------------------
// routing plan, built in LDS by every workgroup in O(P + E)
// ---------------------------------------------------------------------------------------------------------------

// Picks p = t*topk + k are scanned token-major, as the reference builds its jobs (moe_forward, ft_core.h:1343-1349):
//   union of experts in first-appearance order (uexp), one slot per pick grouped by union entry with tokens
//   ascending (uoff / spick), and the index of the reference job every pick lands in (a new job whenever the
//   expert's current job holds 8 tokens), which fixes the order of the weighted sum.
// Ids outside [0, E) are skipped (tier_forward drops sel < 0, ft_tier_ext.cpp:896-898) and counted in bad.
struct LPlan
{
    int* e;       // [P] expert of pick p, -1 if skipped
    int* c;       // [P] occurrence of pick p among its expert's picks (pick order)
    int* rank;    // [P] union rank, valid at an expert's first pick
    int* crank;   // [P] job index, valid at a job's first pick (c % 8 == 0)
    int* spick;   // [P] pick of slot s
    int* uoff;    // [P + 1] slot offsets of the union entries
    int* uexp;    // [P] expert of union entry u
    int* first;   // [E] first pick of expert e
    int* cnt;     // [E] running per-expert count during the scan, then the slot count of union entry u
};

__host__ __device__ constexpr size_t lplan_ints(int P, int E) { return 7 * (size_t)P + 1 + 2 * (size_t)E; }

__device__ inline LPlan lplan_carve(int* base, int P, int E)
{
    LPlan L;
    L.e = base;
    L.c = L.e + P;
    L.rank = L.c + P;
    L.crank = L.rank + P;
    L.spick = L.crank + P;
    L.uoff = L.spick + P;
    L.uexp = L.uoff + P + 1;
    L.first = L.uexp + P;
    L.cnt = L.first + E;
    return L;
}

// Whole workgroup. On return: hdr[0] = U, hdr[1] = slots, hdr[2] = ids outside [0, E); L filled.
__device__ void build_plan(const int64_t* __restrict__ sel, int P, int E, const LPlan& L, int* hdr)
{
    const int t = threadIdx.x, nt = blockDim.x, lane = t & 63;
    for (int e = t; e < E; e += nt) { L.first[e] = 0x7fffffff; L.cnt[e] = 0; }
    if (t == 0) hdr[2] = 0;
    __syncthreads();
    for (int p = t; p < P; p += nt)
    {
        const int64_t e = sel[p];
        const bool ok = e >= 0 && e < E;
        L.e[p] = ok ? (int)e : -1;
        if (ok) atomicMin(&L.first[(int)e], p);
        if (e >= E || e < -1) atomicAdd(&hdr[2], 1);
    }
    __syncthreads();
    if (t < 64)
    {
        // one wave scans the picks in order, 64 at a time: occurrence index from an equal-expert lane mask built with
        // ten ballots (E <= 1024), union ranks and job ranks as ballot prefix sums
        int base_u = 0, base_j = 0;
        const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        for (int p0 = 0; p0 < P; p0 += 64)
        {
            const int p = p0 + lane;
            const int e = p < P ? L.e[p] : -1;
            const bool ok = e >= 0;
            uint64_t eq = __ballot(ok);
#pragma unroll
            for (int b = 0; b < 10; ++b)
            {
                const bool bit = ok && ((e >> b) & 1);
                const uint64_t m = __ballot(bit);
                eq &= bit ? m : ~m;
            }
            const int cin = __popcll(eq & below);
            const int base = ok ? L.cnt[e] : 0;
            const int c = base + cin;
            const bool firstp = ok && c == 0, creator = ok && (c & 7) == 0;
            const uint64_t mf = __ballot(firstp), mc = __ballot(creator);
            if (ok)
            {
                L.c[p] = c;
                if (cin == 0) L.cnt[e] = base + __popcll(eq);   // lowest lane of the group advances the count
            }
            if (firstp)
            {
                const int r = base_u + __popcll(mf & below);
                L.rank[p] = r;
                L.uexp[r] = e;
            }
            if (creator) L.crank[p] = base_j + __popcll(mc & below);
            base_u += __popcll(mf);
            base_j += __popcll(mc);
        }
        if (lane == 0) hdr[0] = base_u;
    }
    __syncthreads();
    const int U = hdr[0];
    // slot counts per union entry (cnt is indexed by expert until here; U <= E entries are rewritten in place only
    // after every thread has read its expert's count; U <= P <= 1024 <= 4 * blockDim.x)
    int mine[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int u = t + i * nt;
        mine[i] = u < U ? L.cnt[L.uexp[u]] : 0;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int u = t + i * nt;
        if (u < U) L.cnt[u] = mine[i];
    }
    __syncthreads();
    if (t < 64)
    {
        int carry = 0;
        for (int u0 = 0; u0 < U; u0 += 64)
        {
            const int u = u0 + lane;
            const int v = u < U ? L.cnt[u] : 0;
            int s = v;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1)
            {
                const int o = __shfl_up(s, d);
                if (lane >= d) s += o;
            }
            if (u < U) L.uoff[u] = carry + s - v;
            carry += __shfl(s, 63);
        }
        if (lane == 0) { L.uoff[U] = carry; hdr[1] = carry; }
    }
    __syncthreads();
    for (int p = t; p < P; p += nt)
    {
        const int e = L.e[p];
        if (e < 0) continue;
        L.spick[L.uoff[L.rank[L.first[e]]] + L.c[p]] = p;
    }
    __syncthreads();
}

// The same plan for P <= 64 picks from one wave, without LDS atomics or intermediate barriers (the decode case):
// lane p holds pick p; all derived quantities are ballot/prefix arithmetic over the wave. first[] is written only for
// the experts present (the only entries read).
// e64_lane: lane p's pick sel[p] (-1 for lanes >= P), already in a register of wave 0
__device__ void build_plan_wave_from(int64_t e64_lane, int P, int E, const LPlan& L, int* hdr)
{
    const int lane = threadIdx.x & 63;
    if (threadIdx.x < 64)
    {
        const int64_t e64 = lane < P ? e64_lane : -1;
        const bool ok = e64 >= 0 && e64 < E;
        const int e = ok ? (int)e64 : -1;
        const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        const uint64_t bad = __ballot(lane < P && (e64 >= E || e64 < -1));
        uint64_t eq = __ballot(ok);
#pragma unroll
        for (int b = 0; b < 10; ++b)
        {
            const bool bit = ok && ((e >> b) & 1);
            const uint64_t m = __ballot(bit);
            eq &= bit ? m : ~m;
        }
        const int c = __popcll(eq & below);
        const bool firstp = ok && c == 0, creator = ok && (c & 7) == 0;
        const uint64_t mf = __ballot(firstp), mc = __ballot(creator);
        const int r = __popcll(mf & below);
        // slot offsets: exclusive prefix of the union entries' pick counts, in first-appearance (= lane) order
        const int v = firstp ? __popcll(eq) : 0;
        int sc = v;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1)
        {
            const int o = __shfl_up(sc, d);
            if (lane >= d) sc += o;
        }
        const int uo = sc - v;
        const int fl = ok ? __builtin_ctzll(eq) : 0;      // lane of the expert's first pick
        const int uo_p = __shfl(uo, fl);
        if (lane < P) L.e[lane] = e;
        if (ok)
        {
            L.c[lane] = c;
            L.spick[uo_p + c] = lane;
        }
        if (firstp)
        {
            L.rank[lane] = r;
            L.uexp[r] = e;
            L.uoff[r] = uo;
            L.first[e] = lane;
        }
        if (creator) L.crank[lane] = __popcll(mc & below);
        const int U = __popcll(mf), S = __shfl(sc, 63);
        if (lane == 0)
        {
            L.uoff[U] = S;
            hdr[0] = U;
            hdr[1] = S;
            hdr[2] = __popcll(bad);
        }
    }
    __syncthreads();
}

__device__ void build_plan_wave(const int64_t* __restrict__ sel, int P, int E, const LPlan& L, int* hdr)
{
    const int lane = threadIdx.x & 63;
    build_plan_wave_from(threadIdx.x < 64 && lane < P ? sel[lane] : -1, P, E, L, hdr);
}

// union entry of pick p's expert and its job index (the job's first pick is the slot 8*floor(c/8) of the entry)
__device__ inline int plan_u(const LPlan& L, int p) { return L.rank[L.first[L.e[p]]]; }
__device__ inline int plan_job(const LPlan& L, int p)
{
    return L.crank[L.spick[L.uoff[plan_u(L, p)] + (L.c[p] & ~7)]];
}

// Publish the plan for the down launch (one workgroup): PlanView arrays plus each token's picks in (job, pick) order
// with their fp32 weights; rows of tokens without a valid pick are written as zeros here (no down workgroup touches
// them; the reference's sum over an empty route is 0). jscr: LDS scratch of P ints (each pick's job, -1 if skipped).
__device__ void publish_plan(const LPlan& L, const int* hdr, int P, int topk, const void* w, int w_half,
                             const PlanView& pv, float* out, int H, const uint64_t* ptrs, int per_slot, int* jscr)
{
    const int t = threadIdx.x, nt = blockDim.x;
    const int U = hdr[0], S = hdr[1];
    // the weights of this thread's picks first (they are stored only at the end; with the loads between the stores
    // below, each would wait for the store before it)
    constexpr int PPT = (MAX_PICKS + 255) / 256;   // picks per thread (both callers run 256 threads)
    float wr[PPT];
#pragma unroll
    for (int i = 0; i < PPT; ++i)
    {
        const int p = min(t + i * nt, P - 1);
        wr[i] = w_half ? h2f_bits(reinterpret_cast<const uint16_t*>(w)[p]) : reinterpret_cast<const float*>(w)[p];
    }
    if (t < 3) pv.hdr[t] = hdr[t];
    for (int u = t; u < U; u += nt)
    {
        const int e = L.uexp[u];
        pv.uexp[u] = e;
        if (!per_slot)
        {
            pv.uptr[2 * u] = ptrs[(size_t)e * 9 + 2];
            pv.uptr[2 * u + 1] = ptrs[(size_t)e * 9 + 8];
        }
    }
    // with per_slot the down launch takes a workgroup per slot: the address table is indexed by slot
    for (int s = t; per_slot && s < S; s += nt)
    {
        const int e = L.e[L.spick[s]];
        pv.uptr[2 * s] = ptrs[(size_t)e * 9 + 2];
        pv.uptr[2 * s + 1] = ptrs[(size_t)e * 9 + 8];
    }
    for (int u = t; u <= U; u += nt) pv.uoff[u] = L.uoff[u];
    for (int s = t; s < S; s += nt) pv.slot_pick[s] = L.spick[s];
    for (int p = t; p < P; p += nt)
    {
        if (L.e[p] < 0)
        {
            pv.pick_slot[p] = -1;
            pv.pick_job[p] = 0x7fffffff;
            jscr[p] = -1;
            continue;
        }
        const int u = plan_u(L, p), s = L.uoff[u] + L.c[p], jb = plan_job(L, p);
        pv.pick_slot[p] = s;
        pv.slot_u[s] = u;
        pv.pick_job[p] = jb;
        jscr[p] = jb;
    }
    __syncthreads();
    // each token's picks in (job, pick) order, a thread per pick: a valid pick's place is the number of the token's
    // valid picks before it in that order; places n..topk-1 of a token with n valid picks are padding (picks past
    // PPT * nt, with fewer than 256 threads, load their weight here)
    for (int i = 0;; ++i)
    {
        const int p = t + i * nt;
        if (p >= P) break;
        float wp = 0.f;
#pragma unroll
        for (int i2 = 0; i2 < PPT; ++i2)
            if (i2 == i) wp = wr[i2];
        if (i >= PPT)
            wp = w_half ? h2f_bits(reinterpret_cast<const uint16_t*>(w)[p]) : reinterpret_cast<const float*>(w)[p];
        const int tk = p / topk, k = p - tk * topk, b = tk * topk, jb = jscr[p];
        int r = 0, n = 0;
        for (int k2 = 0; k2 < topk; ++k2)
        {
            const int j2 = jscr[b + k2];
            n += j2 >= 0 ? 1 : 0;
            r += (j2 >= 0 && (j2 < jb || (j2 == jb && k2 < k))) ? 1 : 0;
        }
        if (jb >= 0)
        {
            pv.tok_slot[b + r] = L.uoff[plan_u(L, p)] + L.c[p];
            pv.tok_w[b + r] = wp;
        }
        if (k >= n)
        {
            pv.tok_slot[b + k] = -1;
            pv.tok_w[b + k] = 0.f;
        }
        if (k == 0)
        {
            pv.tok_npk[tk] = n;
            if (n == 0)
                for (int c = 0; c < H; ++c) out[(size_t)tk * H + c] = 0.f;
        }
    }
}

// The relay launches need no published plan: their workgroups read sel directly, each pick's gate|up workgroup of
// tile-column block 0 publishes the pick's down addresses, and the down launch's combining workgroups form each
// token's job order themselves (relay_combine_list). What is left for the plan block is what no GEMV workgroup
// covers: the address entries of skipped picks (null, so that their down workgroups return) and the output rows of
// tokens without a valid pick (the reference's sum over an empty route is 0).
__device__ void relay_plan_block(const int64_t* __restrict__ sel, int P, int topk, int E, float* out, int H,
                                 uint64_t* uptr, int* flags)
{
    const int t = threadIdx.x, nt = blockDim.x, M = P / topk;
    for (int p = t; p < P; p += nt)
    {
        const int64_t e = sel[p];
        if (e < 0 || e >= E) { uptr[2 * p] = 0; uptr[2 * p + 1] = 0; }
    }
    for (int tk = t; tk < M; tk += nt)
    {
        bool any = false;
        for (int k = 0; k < topk; ++k)
        {
            const int64_t e = sel[(size_t)tk * topk + k];
            any = any || (e >= 0 && e < E);
        }
        flags[tk] = any ? 0 : 1;
    }
    __syncthreads();
    for (int tk = 0; tk < M; ++tk)
        if (flags[tk])
            for (int i = t; i < H; i += nt) out[(size_t)tk * H + i] = 0.f;
}

// The combine list of token tk for a relay down workgroup: the token's valid picks in (job, pick) order, the
// reference's combine order (moe_forward's jobs, ft_core.h:1343-1349 and 1020-1033), as pick indices (the relay's
// slots) with their fp32 weights and svh_down addresses. Jobs are those of build_plan: an expert's picks in pick order,
// a new job at every 8th of them, jobs numbered in the order of their first picks. Wave 0 computes it in registers
// (lane = pick, P <= 64): e64_lane the pick's id, w_lane its weight, svh_lane its expert's svh_down address. Whole
// workgroup (ends with a barrier); writes slot[k], wt[k], sv[k] for k < *npk.
__device__ void relay_combine_list(int64_t e64_lane, float w_lane, uint64_t svh_lane, int P, int E, int topk, int tk,
                                   int* slot, float* wt, uint64_t* sv, int* npk)
{
    if (threadIdx.x < 64)
    {
        const int lane = threadIdx.x;
        const bool ok = lane < P && e64_lane >= 0 && e64_lane < E;
        const int e = ok ? (int)e64_lane : -1;
        // lanes of the same expert: ten ballots on the id bits (E <= 1024)
        uint64_t eq = __ballot(ok);
#pragma unroll
        for (int b = 0; b < 10; ++b)
        {
            const bool bit = ok && ((e >> b) & 1);
            const uint64_t m = __ballot(bit);
            eq &= bit ? m : ~m;
        }
        const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        const int c = __popcll(eq & below);                 // occurrence of the pick among its expert's picks
        const uint64_t mc = __ballot(ok && (c & 7) == 0);  // picks that open a job
        const int crank = __popcll(mc & below);            // job number, at a job's opening pick
        uint64_t m = eq;
        for (int k = 0; k < (c & ~7); ++k) m &= m - 1;      // the opening pick of this pick's job: set bit c & ~7
        const int opener = ok ? __builtin_ctzll(m) : lane;
        const int job = __shfl(crank, opener);
        const bool mine = ok && lane / topk == tk;
        int rank = 0;
        for (int k = 0; k < topk; ++k)
        {
            const int lk = tk * topk + k;
            const int jk = __shfl(job, lk);
            const bool okk = __shfl((int)(ok ? 1 : 0), lk) != 0;
            rank += (okk && (jk < job || (jk == job && lk < lane))) ? 1 : 0;
        }
        if (mine)
        {
            slot[rank] = lane;
            wt[rank] = w_lane;
            sv[rank] = svh_lane;
        }
        const uint64_t mm = __ballot(mine);
        if (lane == 0) *npk = __popcll(mm);
    }
    __syncthreads();
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

// Workgroup barrier that only orders LDS traffic: wait for this wave's LDS operations, then s_barrier (no release
// fence, so outstanding global loads stay in flight).
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// groups of 8 tiles in each wave's LDS ring (3 in flight). Measured against 2..8 groups on MI355X: 3 and 4 are
// fastest at M = 1..4 (a deeper ring puts more loads ahead of the input transform, whose waits cover every load issued
// before it, since the compiler does not count the LDS-direct loads and waits with vmcnt(0)).
constexpr int NGRP = 4;

// bytes per transformed input element in LDS: fp32 with one slot per pass, so that the chain FMAs take fp32 operands,
// else fp16 (eight 5120-wide fp32 inputs would not fit beside the rings)
constexpr int x_lds_elem(int ns) { return ns <= 1 ? 4 : 2; }

// One tile column of one matrix over all TK tile rows for up to NS slots whose transformed inputs sit in lds_x
// ([ns][kdim] in the permuted [tk][j][q] order; fp32 when XF, else fp16 - the values are fp16 either way). Lane
// (j = l/16, n = l%16) carries the reference's accumulator j of output column n.
//
// Each wave streams its own column through a private LDS ring of NG groups of 8 tiles with LDS-direct buffer loads
// (global -> LDS without registers): a group of 8 tiles is 256*K bytes = K dword loads of the 64 lanes, lane l of load
// i fetching byte i*256 + 4l of the group. Group g + NG - 1 is issued before group g is decoded, so NG - 1 groups are
// in flight per wave; the waves of a workgroup never wait for each other. Loads address tile rows < TK only.
// col_base = tile row 0 of the column; tile row r sits at col_base + r * gstride (TK * gstride < 2^31); TK % 8 == 0.
// ring = this wave's NG * 256 * K bytes of LDS. res[s] = the column results (valid in lanes 0..15).
typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt vmcnt(N) (expcnt / lgkmcnt not waited): the LDS-direct loads are not tracked by the compiler, so the
// wait and its ordering against the LDS reads that follow are explicit
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// pre_load() runs before the first NG - 1 groups are requested, pre() after them and before the first is read: the
// caller issues its input loads in pre_load (so waiting for them does not wait for the trellis groups queued behind)
// and fills lds_x in pre (ending with a workgroup barrier), so the input transform overlaps the trellis fetch.
template <int K, int NS, int NG, bool XF, class PreLoad, class Pre>
__device__ __forceinline__ void chain_dma(const uint8_t* __restrict__ col_base, size_t gstride, int TK, int ns,
                                          const void* lds_x, uint8_t* ring, float (&res)[NS], PreLoad&& pre_load,
                                          Pre&& pre)
{
    constexpr int TB = 32 * K, GB = 8 * TB;
    const int lane = threadIdx.x & 63;
    const LaneDec d = lane_dec(lane, K);
    const int j = lane >> 4, n = lane & 15;
    half4 Pm;
#pragma unroll
    for (int r = 0; r < 4; ++r) Pm[r] = (_Float16)((j == (n & 3) && r == (n >> 2)) ? 1.0f : 0.0f);
    const float4v zero = { 0.f, 0.f, 0.f, 0.f };
    uint8_t* cb = const_cast<uint8_t*>(uniform_ptr(col_base));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(cb, (short)0, (int)((size_t)TK * gstride),
                                                                        0x00020000);
    const int gs = (int)gstride;
    int voff[K];
#pragma unroll
    for (int i = 0; i < K; ++i)
    {
        const int byte = i * 256 + lane * 4;
        voff[i] = (byte / TB) * gs + (byte % TB);
    }
    const int ngroups = TK / 8;
    auto issue = [&](int g) {
        uint8_t* dst = ring + (g % NG) * GB;
#pragma unroll
        for (int i = 0; i < K; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + i * 256), 4, voff[i], g * 8 * gs, 0, 0);
    };
    pre_load();
#pragma unroll
    for (int g = 0; g < NG - 1; ++g)
        if (g < ngroups) issue(g);
    pre();
    float acc[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) acc[s] = 0.f;
    const uint16_t* xl = static_cast<const uint16_t*>(lds_x) + j * 4;
    const float* xlf = static_cast<const float*>(lds_x) + j * 4;
    for (int g = 0; g < ngroups; ++g)
    {
        if (g + NG - 1 < ngroups)
        {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // reads of the slot being refilled are done
            issue(g + NG - 1);
            wait_vmcnt<(NG - 1) * K>();                          // group g has landed
        }
        else
            wait_vmcnt<0>();
        const uint8_t* sl = ring + (g % NG) * GB;
#pragma unroll
        for (int h = 0; h < 8; h += 8)   // all 8 tiles of the group per block (more independent work for a lone wave)
        {
            float4v cw[8];
#pragma unroll
            for (int rr = 0; rr < 8; ++rr)
            {
                const uint8_t* tp = sl + (h + rr) * TB;
                const uint32_t hi = *reinterpret_cast<const uint32_t*>(tp + d.o0);
                const uint32_t lo = *reinterpret_cast<const uint32_t*>(tp + d.o1);
                cw[rr] = __builtin_amdgcn_mfma_f32_16x16x16f16(Pm, decode4<K>(hi, lo, d.sh), zero, 0, 0, 0);
            }
#pragma unroll
            for (int s = 0; s < NS; ++s)
            {
                if (s == 0 || s < ns)
                {
                    float a = acc[s];
                    float4v xf[8];
                    if constexpr (XF)
                    {
                        // fp32 operands: the FMAs are v_fmac_f32, which issue at twice the rate of the
                        // mixed-precision v_fma_mix_f32 an fp16 operand needs; the 8 reads go out together
#pragma unroll
                        for (int rr = 0; rr < 8; ++rr)
                            xf[rr] = *reinterpret_cast<const float4v*>(xlf + ((size_t)s * TK + g * 8 + h + rr) * 16);
                    }
#pragma unroll
                    for (int rr = 0; rr < 8; ++rr)
                    {
                        const int tk = g * 8 + h + rr;
                        if constexpr (XF)
                        {
                            a = __builtin_fmaf(cw[rr][0], xf[rr][0], a);
                            a = __builtin_fmaf(cw[rr][1], xf[rr][1], a);
                            a = __builtin_fmaf(cw[rr][2], xf[rr][2], a);
                            a = __builtin_fmaf(cw[rr][3], xf[rr][3], a);
                        }
                        else
                        {
                            const half4 xv = *reinterpret_cast<const half4*>(xl + ((size_t)s * TK + tk) * 16);
                            a = __builtin_fmaf(cw[rr][0], (float)xv[0], a);
                            a = __builtin_fmaf(cw[rr][1], (float)xv[1], a);
                            a = __builtin_fmaf(cw[rr][2], (float)xv[2], a);
                            a = __builtin_fmaf(cw[rr][3], (float)xv[3], a);
                        }
                    }
                    acc[s] = a;
                }
            }
        }
    }
#pragma unroll
    for (int s = 0; s < NS; ++s)
    {
        const float a1 = __shfl(acc[s], n + 16), a2 = __shfl(acc[s], n + 32), a3 = __shfl(acc[s], n + 48);
        res[s] = (acc[s] + a1) + (a2 + a3);
    }
}

// One tile column of one matrix for one slot, its groups of 8 tile rows shared out over RW waves of the workgroup: the
// wave with relay index r streams and decodes groups r, r + RW, r + 2 RW, ..., and the column's accumulators pass from
// wave to wave through relay (64 floats in LDS) in group order, so every accumulator is still one chain of fused
// multiply-adds over the tile rows in the reference's order.
// Phase ph: each wave decodes and transposes its group g = ph * RW + r, waits until the column's turn counter (LDS)
// reaches g, reads the accumulators of group g - 1, runs the group's 32 FMAs, writes them back and moves the counter
// to g + 1 (release/acquire at workgroup scope). Only the wave of the next group waits, and each wave decodes its
// next group before it waits; workgroup barriers coupling all waves at every turn measured 1-7 us slower at M=1..4.
// The trellis streams through registers: each wave keeps its next PF groups in flight as 16-byte buffer loads (lane l
// of load i holds byte 16 (64 i + l) of the group: tile (64 i + l) / 2K, bytes 16 ((64 i + l) % 2K) onward) and writes
// a group into its single LDS slot (8 tiles, tile-major) right before decoding it. LDS operations of one wave complete
// in issue order, so the slot is rewritten only after the previous group's reads; the waits for the loads are the
// compiler's own (registers it tracks). lds_x: the slot's transformed inputs as fp32 in the permuted [tk][j][q] order,
// filled by pre() (which ends with a workgroup barrier) while the first groups are in flight.
// Returns the column results (valid in lanes 0..15 of every relay wave of the column).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Work item of relay launch block b (a grid of relay_blocks(items, RW) blocks): items are (entry, column block),
// column blocks fastest, and each run of RW adjacent column blocks (4 tile columns, whole 128-byte lines of every tile
// row) goes to one XCD (XCD = block index mod 8), the runs dealt round-robin over the 8 XCDs. Blocks past the items
// return -1. Adjacent column blocks of fewer than 4 tile columns share lines; on different XCDs each L2 would fetch
// them (measured 1.38x the algorithmic bytes of the gate|up launch with 2 columns per workgroup).
__device__ __forceinline__ long relay_item(long b, int RW, long items)
{
    const long xcd = b % 8, j = b / 8;
    const long item = ((j / RW) * 8 + xcd) * RW + j % RW;
    return item < items ? item : -1;
}
__host__ __device__ constexpr long relay_blocks(long items, int RW)
{
    return (items / RW + 7) / 8 * 8 * RW;
}

// Bounded wait for a relay turn: polls `turn` (workgroup-scope acquire) until it reaches g, at most spin_max polls
// rounded up to a multiple of 8. Returns false when the bound ran out first; the caller then counts the expiry in the
// context's status word, which the host reads with gfl_ctx_check (the call's outputs are then wrong, and reported as
// such). spin_max = 0 polls never and always expires: the host sets it only to test that reporting path.
__device__ __forceinline__ bool wait_turn(const int* turn, int g, int spin_max)
{
    // polls in runs of 8 with the bound checked once per run: a hand-off is seen within a poll's LDS read and one
    // s_sleep, with no loop bookkeeping between polls (the relay's serial chain waits on every group's turn)
    for (int spin = 0; spin < spin_max; spin += 8)
    {
#pragma unroll
        for (int u = 0; u < 8; ++u)
        {
            if (__hip_atomic_load(turn, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= g) return true;
            __builtin_amdgcn_s_sleep(1);
        }
    }
    return false;
}

__device__ __forceinline__ void count_expiry(int* status)
{
    __hip_atomic_fetch_add(&status[GFL_STATUS_RELAY_EXPIRED], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int K, int PF, int RW, class PreLoad, class Pre>
__device__ __forceinline__ float chain_relay(const uint8_t* __restrict__ col_base, size_t gstride, int TK,
                                             const float* lds_x, uint8_t* slot, float* relay, int* turn, int r,
                                             int* status, int spin_max, int prio, PreLoad&& pre_load, Pre&& pre)
{
    constexpr int TB = 32 * K, CH = 2 * K, NCH = 8 * CH, NLD = (NCH + 63) / 64;   // 16-byte chunks
    const int lane = threadIdx.x & 63;
    const LaneDec d = lane_dec(lane, K);
    const int j = lane >> 4, n = lane & 15;
    half4 Pm;
#pragma unroll
    for (int i = 0; i < 4; ++i) Pm[i] = (_Float16)((j == (n & 3) && i == (n >> 2)) ? 1.0f : 0.0f);
    const float4v zero = { 0.f, 0.f, 0.f, 0.f };
    uint8_t* cb = const_cast<uint8_t*>(uniform_ptr(col_base));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(cb, (short)0, (int)((size_t)TK * gstride),
                                                                        0x00020000);
    const int gs = (int)gstride;
    int voff[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i)
    {
        const int q = 64 * i + lane;
        voff[i] = q < NCH ? (q / CH) * gs + (q % CH) * 16 : 0;
    }
    const int ngroups = TK / 8, nph = (ngroups + RW - 1) / RW;
    // every phase issues the same loads (group index clamped to the last group, which stays in bounds), so the
    // compiler's wait before writing a group to LDS counts exactly the PF - 1 younger groups
    u32x4 buf[PF][NLD];
    auto load = [&](u32x4 (&b)[NLD], int ph) {
        const int g = min(ph * RW + r, ngroups - 1);
#pragma unroll
        for (int i = 0; i < NLD; ++i)
            b[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff[i], g * 8 * gs, 0);   // lanes past the group: chunk 0
    };
    pre_load();
#pragma unroll
    for (int k = 0; k < PF; ++k) load(buf[k], k);
    float acc = 0.f;
    // every turn wait ended in time; an expiry is counted once, after the loop, so the hand-off path of each group
    // carries no branch around the status word's atomic
    bool waits_ok = true;
    const int nphp = (nph + PF - 1) / PF * PF;   // phases padded to whole rounds of PF (the padding has no work)
    for (int ph0 = 0; ph0 < nphp; ph0 += PF)
    {
        // prio: the wave's issue priority falls from 3 to 0 over the quarters of its phases. A SIMD issues its
        // oldest ready wave first; with 2 or 3 waves per SIMD the oldest then finish early and the youngest runs its
        // last stretch alone, at about half the rate of two waves sharing the SIMD. Waves that are ahead yield to
        // those behind, so the waves of a SIMD end together.
        if (prio)
        {
            const int q4 = (4 * ph0) / nphp;
            if (q4 == 0) __builtin_amdgcn_s_setprio(3);
            else if (q4 == 1) __builtin_amdgcn_s_setprio(2);
            else if (q4 == 2) __builtin_amdgcn_s_setprio(1);
            else __builtin_amdgcn_s_setprio(0);
        }
#pragma unroll
        for (int k = 0; k < PF; ++k)
        {
            const int ph = ph0 + k;
            const int g = ph * RW + r;
            const bool mine = ph < nph && g < ngroups;
            float4v cw[8], xf[8];
            // the input transform (ending with a workgroup barrier) first: at the launch's start every workgroup's
            // first trellis groups queue behind one another in HBM, and the inputs (x from L2, suh shared by the
            // expert's workgroups) land sooner, so the transform fills that wait (before the first group's decode it
            // measured 1.1 us faster at config 1 M=1 than after it)
            if (ph == 0) pre();
            // written in every phase, padding ones included (the slot is this wave's own and only its own decode
            // reads it): with the write under the phase's branch, the compiler's wait before it also covered the
            // younger of the groups in flight
#pragma unroll
            for (int i = 0; i < NLD; ++i)
                if (64 * i + lane < NCH) *reinterpret_cast<u32x4*>(slot + (64 * i + lane) * 16) = buf[k][i];
            load(buf[k], ph + PF);
            if (mine)
            {
#pragma unroll
                for (int rr = 0; rr < 8; ++rr)
                {
                    const uint8_t* tp = slot + rr * TB;
                    const uint32_t hi = *reinterpret_cast<const uint32_t*>(tp + d.o0);
                    const uint32_t lo = *reinterpret_cast<const uint32_t*>(tp + d.o1);
                    cw[rr] = __builtin_amdgcn_mfma_f32_16x16x16f16(Pm, decode4<K>(hi, lo, d.sh), zero, 0, 0, 0);
                }
            }
            if (mine)
            {
#pragma unroll
                for (int rr = 0; rr < 8; ++rr)
                    xf[rr] = *reinterpret_cast<const float4v*>(lds_x + ((size_t)g * 8 + rr) * 16 + j * 4);
            }
            if (mine)
            {
                if (RW > 1 && g > 0)
                {
                    // the turn of group g: the wave of group g - 1 has written its accumulators (bounded wait: that
                    // wave is resident and waits only for groups before its own). With one wave per column the
                    // accumulators stay in registers.
                    waits_ok &= wait_turn(turn, g, spin_max);
                    acc = relay[lane];
                }
#pragma unroll
                for (int rr = 0; rr < 8; ++rr)
                {
                    acc = __builtin_fmaf(cw[rr][0], xf[rr][0], acc);
                    acc = __builtin_fmaf(cw[rr][1], xf[rr][1], acc);
                    acc = __builtin_fmaf(cw[rr][2], xf[rr][2], acc);
                    acc = __builtin_fmaf(cw[rr][3], xf[rr][3], acc);
                }
                if (RW > 1)
                {
                    relay[lane] = acc;
                    __hip_atomic_store(turn, g + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
            }
        }
    }
    if (prio) __builtin_amdgcn_s_setprio(0);
    wait_vmcnt<0>();   // the padding's clamped prefetches
    if (RW > 1)
    {
        // the last group's accumulators
        waits_ok &= wait_turn(turn, ngroups, spin_max);
        acc = relay[lane];
        if (!waits_ok && lane == 0) count_expiry(status);
    }
    const float a1 = __shfl(acc, n + 16), a2 = __shfl(acc, n + 32), a3 = __shfl(acc, n + 48);
    return (acc + a1) + (a2 + a3);
}

// MFMA-accumulate form of the column GEMV (mode GFL_MODE_MFMA): tile groups [g0, g1) of one tile column for up to 16
// slots whose transformed inputs of 128-blocks g0..g1-1 sit in lds_x as fp16 in the MFMA input layout (gp_perm_pos,
// relative to block g0; xs elements per slot).
// Each pair of tile rows is one v_mfma_f32_16x16x32_f16 whose B slice is the decoded weights as decode4 leaves them
// (lane 16q + n: column n, rows 2q + {0, 1, 8, 9} of both tiles) and whose A row m is slot m (rows >= ns read slot 0;
// their sums are not used). Returns D: lane l holds slot 4(l/16) + i, column l % 16, in element i. The weights and
// every transform are the reference's; only the sums over the hidden dimension are formed in MFMA order instead of
// the EXACT chain order. Streaming is chain_dma's: a private LDS ring of NG groups per wave, NG - 1 in flight.
template <int K, int NG, class PreLoad, class Pre>
__device__ __forceinline__ float4v chain_mf(const uint8_t* __restrict__ col_base, size_t gstride, int TK, int g0,
                                            int g1, const uint16_t* lds_x, int xs, int ns, uint8_t* ring,
                                            PreLoad&& pre_load, Pre&& pre)
{
    constexpr int TB = 32 * K, GB = 8 * TB;
    const int lane = threadIdx.x & 63;
    const LaneDec d = lane_dec(lane, K);
    const int q = lane >> 4, i16 = lane & 15;
    uint8_t* cb = const_cast<uint8_t*>(uniform_ptr(col_base));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(cb, (short)0, (int)((size_t)TK * gstride),
                                                                        0x00020000);
    const int gs = (int)gstride;
    int voff[K];
#pragma unroll
    for (int i = 0; i < K; ++i)
    {
        const int byte = i * 256 + lane * 4;
        voff[i] = (byte / TB) * gs + (byte % TB);
    }
    const int ng = g1 - g0;
    auto issue = [&](int gi) {
        uint8_t* dst = ring + (gi % NG) * GB;
#pragma unroll
        for (int i = 0; i < K; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + i * 256), 4, voff[i], (g0 + gi) * 8 * gs, 0,
                                                     0);
    };
    pre_load();
#pragma unroll
    for (int gi = 0; gi < NG - 1; ++gi)
        if (gi < ng) issue(gi);
    pre();
    float4v acc = { 0.f, 0.f, 0.f, 0.f };
    const uint16_t* xa = lds_x + (size_t)(i16 < ns ? i16 : 0) * xs + q * 32;
    for (int gi = 0; gi < ng; ++gi)
    {
        if (gi + NG - 1 < ng)
        {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // reads of the slot being refilled are done
            issue(gi + NG - 1);
            wait_vmcnt<(NG - 1) * K>();                           // group gi has landed
        }
        else
            wait_vmcnt<0>();
        const uint8_t* sl = ring + (gi % NG) * GB;
        const uint16_t* xg = xa + (size_t)gi * 128;   // the group's 8 tile rows are 128-block g0 + gi
        uint32_t wd[8][2];
#pragma unroll
        for (int rr = 0; rr < 8; ++rr)
        {
            wd[rr][0] = *reinterpret_cast<const uint32_t*>(sl + rr * TB + d.o0);
            wd[rr][1] = *reinterpret_cast<const uint32_t*>(sl + rr * TB + d.o1);
        }
#pragma unroll
        for (int rp = 0; rp < 4; ++rp)
        {
            const half8 A = *reinterpret_cast<const half8*>(xg + rp * 8);
            const half4 B0 = decode4<K>(wd[2 * rp][0], wd[2 * rp][1], d.sh);
            const half4 B1 = decode4<K>(wd[2 * rp + 1][0], wd[2 * rp + 1][1], d.sh);
            const half8 B = { B0[0], B0[1], B0[2], B0[3], B1[0], B1[1], B1[2], B1[3] };
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, acc, 0, 0, 0);
        }
    }
    return acc;
}

// ---------------------------------------------------------------------------------------------------------------
// gate|up launch
// ---------------------------------------------------------------------------------------------------------------

constexpr int GU_NW = 4;    // waves (tile columns) per gate|up workgroup: 64 outputs
constexpr int GU_PR = 3;    // input-transform rounds (4 blocks per wave each) a gate|up wave keeps loads in flight for
constexpr int DN_NW = 8;    // waves per down workgroup: one 128-output block, out_block fused

struct GuArgs
{
    const uint64_t* ptrs;      // [E][9] layer table
    const int64_t* sel;
    const void* w;
    int w_half, P, topk, E, H, I;
    int mat_base;              // matrix of blockIdx.y == 0 (0 gate, 1 up)
    const uint16_t* x;         // [M][H] fp16
    float* ygu;                // [2][cap][I] (MF: [2 halves][2][cap][I])
    uint16_t* xtd;             // [cap][I] down input, permuted
    int* act_cnt;              // [cap][I/128] last-one counters (zero between calls)
    const float* silu_tab;
    float act_limit;
    PlanView pv;               // written by workgroup (0, 0)
    float* out;                // [M][H] (rows of tokens without picks zeroed here)
    int nmat_total;            // gate|up workgroups covering one 128-block
    int ns_cap;                // slots per pass the LDS allocation holds (<= NS)
    int per_slot;              // workgroups per slot (one pass each) instead of per union entry (NS == 1 only)
    int mf;                    // MFMA-accumulate mode: down inputs written in the MFMA input layout
    int nmat_launch;           // matrices of this launch (the relay launches' item count)
    int* status;               // the context's status words (relay waits that expired)
    int spin_max;              // bound of a relay turn wait, in polls
    int prio;                  // relay launches: waves lower their issue priority as they progress (chain_relay)
    int nsh;                   // relay launches: shared-expert picks P .. P + nsh - 1 (token p - P, expert row E,
                               // weight 1), one per token, or 0
    int gplan;                 // the routing plan was published to pv by plan_kernel before this launch: workgroups
                               // read their entries from pv instead of each building the plan in LDS
};

__device__ __forceinline__ float ld_agent(const float* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Last-one counters hand data between workgroups. Everything handed over is written with st_agent and read with
// ld_agent: device-scope (sc1) accesses, performed at the level where all XCDs see them, never served from a stale
// line of one XCD's L2. What the hand-over needs is order: every wave that stored data for the finisher runs
// release_agent() before the workgroup barrier that precedes the counter update, so its stores have completed (the
// barrier alone does not wait for them); the finisher issues its loads only after the counter value came back.
// The generic agent-scope release/acquire fences would add an L2 write-back and invalidate per hand-over, which
// none of these accesses needs (and which costs more than the whole GEMV at decode sizes).
__device__ __forceinline__ void release_agent()
{
    __builtin_amdgcn_s_waitcnt(0x0F70);   // s_waitcnt vmcnt(0) (expcnt and lgkmcnt at their maxima: no wait)
}

// fwd_phase phase 1 for one 128-block b of union entry u (ft_core.h:974-991): out_block of gate and up,
// r16(act_mul), down prep_block, stored permuted as the down GEMV input
__device__ void act_block(const GuArgs& a, int e, int s_begin, int s_end, int b)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    const gptr<uint16_t> svh_g = gaddr<uint16_t>(a.ptrs[(size_t)e * 9 + 4]);
    const gptr<uint16_t> svh_u = gaddr<uint16_t>(a.ptrs[(size_t)e * 9 + 6]);
    const gptr<uint16_t> suh_d = gaddr<uint16_t>(a.ptrs[(size_t)e * 9 + 7]);
    const int cap = a.pv.cap_slots;
    for (int s = s_begin + wave; s < s_end; s += nw)
    {
        const float* yg = a.ygu + (size_t)s * a.I + b * 128;
        const float* yu = a.ygu + (size_t)cap * a.I + (size_t)s * a.I + b * 128;
        float g0 = ld_agent(&yg[lane]), g1 = ld_agent(&yg[lane + 64]);
        float u0 = ld_agent(&yu[lane]), u1 = ld_agent(&yu[lane + 64]);
        if (a.mf)
        {
            // MF: the upper halves of the tile rows, added to the lower halves' sums
            const size_t hoff = (size_t)2 * cap * a.I;
            g0 = g0 + ld_agent(&yg[hoff + lane]);
            g1 = g1 + ld_agent(&yg[hoff + lane + 64]);
            u0 = u0 + ld_agent(&yu[hoff + lane]);
            u1 = u1 + ld_agent(&yu[hoff + lane + 64]);
        }
        out_block_wave(g0, g1, h2f_bits(svh_g[b * 128 + lane]), h2f_bits(svh_g[b * 128 + lane + 64]));
        out_block_wave(u0, u1, h2f_bits(svh_u[b * 128 + lane]), h2f_bits(svh_u[b * 128 + lane + 64]));
        float a0 = r16(act_mul(g0, u0, a.act_limit, a.silu_tab)), a1 = r16(act_mul(g1, u1, a.act_limit, a.silu_tab));
        prep_block_wave(a0, a1, h2f_bits(suh_d[b * 128 + lane]), h2f_bits(suh_d[b * 128 + lane + 64]));
        uint16_t* dst = a.xtd + (size_t)s * a.I;
        dst[a.mf ? gp_perm_pos(b, lane) : perm_pos(b, lane)] = (uint16_t)f2h_bits(a0);
        dst[a.mf ? gp_perm_pos(b, lane + 64) : perm_pos(b, lane + 64)] = (uint16_t)f2h_bits(a1);
    }
}

// The routing plan of a call, built once and published to pv before the gate|up launch (calls above 64 picks
// outside the relay launches). Each of the launch's thousands of workgroups building the whole plan itself (one wave
// scanning every pick with ballots while the others wait) measured 2.6% of the layer at M = 12..16 and 6.4% at
// M = 32..64 (config 1, a second build per workgroup), and its LDS (17 KB at 512 picks) held the gate|up launch to 3
// workgroups per CU. One workgroup of 256 threads; dynamic LDS: lplan_ints(P, E) + P ints.
__global__ __launch_bounds__(GU_NW * 64) void plan_kernel(GuArgs a)
{
    extern __shared__ __align__(16) uint8_t lds_raw[];
    __shared__ int hdr[4];
    const LPlan L = lplan_carve(reinterpret_cast<int*>(lds_raw), a.P, a.E);
    if (a.P <= 64) build_plan_wave(a.sel, a.P, a.E, L, hdr);
    else build_plan(a.sel, a.P, a.E, L, hdr);
    publish_plan(L, hdr, a.P, a.topk, a.w, a.w_half, a.pv, a.out, a.H, a.ptrs, a.per_slot,
                 reinterpret_cast<int*>(lds_raw) + lplan_ints(a.P, a.E));
}

// Grid: (umax * I/64 + 1, nmat). Workgroup = 4 waves = 64 outputs of one matrix of one routed expert, all its
// slots; the last workgroup of row 0 publishes the plan. With per_slot the grid is (P * I/64 + 1, nmat) and a
// workgroup takes one slot: an expert picked by several tokens is streamed once per slot, in parallel, instead of in
// passes one after another.
// MF (MFMA-accumulate mode): a workgroup covers 4 tile columns over one half of the tile rows (so it transforms only
// that half of the inputs), for all slots of its union entry in passes of up to 16; the two halves' partial sums go
// to ygu[half] and the SwiGLU stage adds them (half 0 + half 1).
// Occupancy hint: 3 waves per SIMD for the EXACT kernel with one slot per pass (its batched fp32 input reads need up
// to 168 VGPRs; at 128 the compiler spills), else 4.
template <int K, int NS, bool MF>
__global__ __launch_bounds__(GU_NW * 64) __attribute__((amdgpu_waves_per_eu(K == 5 || (NS == 1 && !MF) ? 3 : 4))) void
gu_kernel(GuArgs a)
{
    constexpr int NW = GU_NW, TB = 32 * K;
    extern __shared__ __align__(16) uint8_t lds_raw[];
    __shared__ int hdr[4];
    __shared__ int s_last;
    constexpr int RB = NGRP * 8 * TB;                                                 // ring bytes per wave
    uint8_t* rings = lds_raw;                                                         // [NW][RB]
    constexpr bool XF = !MF && x_lds_elem(NS) == 4;
    constexpr int XE = MF ? 2 : x_lds_elem(NS);
    void* lds_x = lds_raw + NW * RB;                                                  // [ns_cap][H] permuted
    // [ns_cap][H] elements, MF: [ns_cap][H / 2] (one half of the 128-blocks)
    int* plan_mem = reinterpret_cast<int*>(lds_raw + NW * RB + (size_t)a.ns_cap * a.H * XE / (MF ? 2 : 1));
    const int TN = a.I / 16, TK = a.H / 16, ncb = TN / NW;
    const LPlan L = lplan_carve(plan_mem, a.P, a.E);
    if (!a.gplan)
    {
        if (a.P <= 64) build_plan_wave(a.sel, a.P, a.E, L, hdr);
        else build_plan(a.sel, a.P, a.E, L, hdr);
    }
    if (blockIdx.x == gridDim.x - 1)
    {
        // the grid's extra workgroup publishes the plan for the down launch (no GEMV work of its own)
        if (blockIdx.y == 0 && !a.gplan)
            publish_plan(L, hdr, a.P, a.topk, a.w, a.w_half, a.pv, a.out, a.H, a.ptrs, a.per_slot,
                         reinterpret_cast<int*>(rings));   // the rings (>= 8 KB) are free in this workgroup
        return;
    }

    // union entry (or slot with per_slot), column block, and with MF the half of the tile rows (adjacent workgroups)
    const int nper = MF ? 2 * ncb : ncb;
    const int ent = blockIdx.x / nper, cb = (blockIdx.x % nper) / (MF ? 2 : 1), hf = MF ? blockIdx.x & 1 : 0;
    if (ent >= (a.gplan ? a.pv.hdr[a.per_slot ? 1 : 0] : hdr[a.per_slot ? 1 : 0])) return;
    const int u = a.per_slot ? (a.gplan ? a.pv.slot_u[ent] : plan_u(L, L.spick[ent])) : ent;
    const int mat = a.mat_base + blockIdx.y;              // 0 gate, 1 up
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, n = lane & 15;
    const int wid = __builtin_amdgcn_readfirstlane(wave);
    const int e = a.gplan ? a.pv.uexp[u] : L.uexp[u];
    const uint8_t* tr = reinterpret_cast<const uint8_t*>(a.ptrs[(size_t)e * 9 + mat]);
    const gptr<uint16_t> suh = gaddr<uint16_t>(a.ptrs[(size_t)e * 9 + 3 + 2 * mat]);
    const int s_begin = a.per_slot ? ent : (a.gplan ? a.pv.uoff[u] : L.uoff[u]);
    const int s_end = a.per_slot ? ent + 1 : (a.gplan ? a.pv.uoff[u + 1] : L.uoff[u + 1]);
    const size_t gstride = (size_t)TN * TB;
    const int t = cb * NW + wave;                         // this wave's tile column
    const uint8_t* col = tr + (size_t)t * TB;
    float* ybase = a.ygu + (size_t)(2 * hf + mat) * a.pv.cap_slots * a.I;
    const int ngr = TK / 8, g0 = hf ? ngr / 2 : 0, g1 = MF && !hf ? ngr / 2 : ngr;   // this workgroup's 128-blocks
    const int xs = (g1 - g0) * 128;                                                    // LDS input row (elements)

    const int nsp = MF ? max(1, min(16, a.ns_cap)) : NS == 1 ? 1 : max(1, min(NS, a.ns_cap));
    for (int c0 = s_begin; c0 < s_end; c0 += nsp)
    {
        const int ns = NS == 1 && !MF ? 1 : min(nsp, s_end - c0);   // >= 1 (c0 < s_end)
        lds_barrier();   // previous pass done with lds_x (and red)
        float res[NS];
        // input transform of the pass's tokens into LDS (prep_block, ft_core.h:97-102): each 16-lane row of a wave
        // takes one (slot, 128-block) item, 8 elements per lane; the first GU_PR rounds of items are loaded before the
        // trellis groups are requested
        const int nblk = g1 - g0, nit = ns * nblk, rl = lane >> 4, li = lane & 15;
        uint4 xv[GU_PR], sv[GU_PR];
        auto load_round = [&](int r, int k) {
            const int it = min((r * NW + wave) * 4 + rl, nit - 1);
            const int s = it / nblk, b = g0 + it % nblk;
            const int pk = a.gplan ? a.pv.slot_pick[c0 + s] : L.spick[c0 + s];
            xv[k] = *reinterpret_cast<const uint4*>(a.x + (size_t)(pk / a.topk) * a.H + b * 128 + li * 8);
            sv[k] = gld16(suh, b * 128 + li * 8);
        };
        auto prep_round = [&](int r, int k) {
            const int it = (r * NW + wave) * 4 + rl;
            float v[8];
            prep_block_row_p(v, xv[k], sv[k]);
            if (it < nit)
            {
                // elements 8li..8li+7 of block b: tile row li/2, accumulators j0 = 2(li&1) and j0 + 1, q = k/2
                const int s = it / nblk, b = it % nblk, tk = b * 8 + (li >> 1), j0 = 2 * (li & 1);   // b from g0
                const size_t pos = (size_t)s * a.H + (tk * 4 + j0) * 4;
                if constexpr (MF)
                {
                    uint32_t o[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) o[q] = f2h2_bits(v[2 * q], v[2 * q + 1]);
                    gp_store_row(static_cast<uint16_t*>(lds_x) + (size_t)s * xs, b, li, o);
                }
                else if constexpr (XF)
                {
                    float* dst = static_cast<float*>(lds_x) + pos;
                    float4v e0, e1;
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                    {
                        e0[q] = h2f_bits((uint16_t)f2h_bits(v[2 * q]));
                        e1[q] = h2f_bits((uint16_t)f2h_bits(v[2 * q + 1]));
                    }
                    *reinterpret_cast<float4v*>(dst) = e0;
                    *reinterpret_cast<float4v*>(dst + 4) = e1;
                }
                else
                {
                    uint16_t* dst = static_cast<uint16_t*>(lds_x) + pos;
                    uint2 e0, e1;
                    e0.x = f2h2_bits(v[0], v[2]);
                    e0.y = f2h2_bits(v[4], v[6]);
                    e1.x = f2h2_bits(v[1], v[3]);
                    e1.y = f2h2_bits(v[5], v[7]);
                    *reinterpret_cast<uint2*>(dst) = e0;
                    *reinterpret_cast<uint2*>(dst + 4) = e1;
                }
            }
        };
        const int nr = (nit + 4 * NW - 1) / (4 * NW);   // rounds of 4 * NW items
        auto pre_load = [&] {
#pragma unroll
            for (int k = 0; k < GU_PR; ++k)
                if (k < nr) load_round(k, k);
        };
        auto pre = [&] {
            for (int r0 = 0; r0 < nr; r0 += GU_PR)
            {
                if (r0 > 0)
                {
#pragma unroll
                    for (int k = 0; k < GU_PR; ++k)
                        if (r0 + k < nr) load_round(r0 + k, k);
                }
#pragma unroll
                for (int k = 0; k < GU_PR; ++k)
                    if (r0 + k < nr) prep_round(r0 + k, k);
            }
            lds_barrier();   // lds_x complete
        };
        if constexpr (MF)
        {
            const float4v acc = chain_mf<K, NGRP>(col, gstride, TK, g0, g1, static_cast<const uint16_t*>(lds_x), xs,
                                                  ns, rings + wid * RB, pre_load, pre);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
            {
                const int m = 4 * (lane >> 4) + rr;
                if (m < ns)
                    __hip_atomic_store(&ybase[(size_t)(c0 + m) * a.I + t * 16 + n], acc[rr], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        else
        {
            chain_dma<K, NS, NGRP, XF>(col, gstride, TK, ns, lds_x, rings + wid * RB, res, pre_load, pre);
#pragma unroll
            for (int s = 0; s < NS; ++s)
                if (s < ns && lane < 16)
                    __hip_atomic_store(&ybase[(size_t)(c0 + s) * a.I + t * 16 + n], res[s], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // the last of the workgroups covering this 128-block (its gate and up halves) runs the SwiGLU stage for it
    release_agent();
    __syncthreads();
    const int blk = (cb * NW * 16) / 128;
    if (threadIdx.x == 0)
    {
        int* ctr = a.act_cnt + ((size_t)ent * (a.I / 128) + blk) * CNT_STRIDE;
        const int old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == a.nmat_total - 1;
        if (s_last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (s_last) act_block(a, e, s_begin, s_end, blk);
}

// ---------------------------------------------------------------------------------------------------------------
// down launch
// ---------------------------------------------------------------------------------------------------------------

struct DnArgs
{
    const uint64_t* ptrs;
    int topk, H, I;
    PlanView pv;
    const uint16_t* xtd;       // [cap][I]
    float* yd;                 // [cap][H] expert outputs after out_block
    int* out_cnt;              // [tokens][H/128] last-one counters (zero between calls)
    int* blk_cnt;              // [cap][H/128] half-block counters of the one-slot-per-pass launch (zero between
                               // calls)
    float* out;                // [M][H]
    int ns_cap;                // slots per pass the LDS allocation holds (<= NS)
    int per_slot;              // workgroups per slot (one pass each), as the gate|up launch
    int pv_picks;              // picks of the call (the relay down launch's item count)
    int* status;               // the context's status words (relay waits that expired)
    int spin_max;              // bound of a relay turn wait, in polls
    int prio;                  // relay launches: waves lower their issue priority as they progress (chain_relay)
    int nsh;                   // relay launches: shared-expert picks after the routed ones, as in GuArgs
    const int64_t* sel;        // [P] picks (relay launches: slot = pick)
    const void* w;             // [P] routing weights, fp16 (w_half) or fp32
    int w_half, E;
};

// Grid: umax * H/128. Workgroup = 8 waves = one 128-output block of one routed expert, all its slots (with per_slot:
// P * H/128, one slot each).
// MF: the GEMV accumulates with MFMAs (chain_mf), for up to 16 slots per pass.
// One slot per pass (EXACT): 4-wave workgroups on half a 128-block each (HB), so that at M=1 the 2,560 down columns
// spread over the CUs in units of 4 (at most 3 columns per SIMD) instead of 8; the two halves' raw sums meet in yd and
// the second to finish runs out_block on the block.
template <int K, int NS, bool MF>
__global__ __launch_bounds__((NS == 1 && !MF ? DN_NW / 2 : DN_NW) * 64)
__attribute__((amdgpu_waves_per_eu(K == 5 || NS == 8 ? 3 : 4))) void down_kernel(DnArgs a)
{
    constexpr bool HB = NS == 1 && !MF;
    constexpr int NW = HB ? DN_NW / 2 : DN_NW, TB = 32 * K;
    extern __shared__ __align__(16) uint8_t lds_raw[];
    __shared__ int s_last[NS];
    __shared__ int c_tok[NS], c_npk[NS], c_slot[NS][MAX_TOPK];
    __shared__ float c_w[NS][MAX_TOPK];
    constexpr int RB = NGRP * 8 * TB;                                                  // ring bytes per wave
    uint8_t* rings = lds_raw;                                                          // [NW][RB]
    constexpr bool XF = !MF && x_lds_elem(NS) == 4;
    constexpr int XE = MF ? 2 : x_lds_elem(NS);
    void* lds_x = lds_raw + NW * RB;                                                   // [ns_cap][I]
    float* lds_y = reinterpret_cast<float*>(lds_raw + NW * RB + (size_t)a.ns_cap * a.I * XE);   // [ns_cap][128]
    const int TN = a.H / 16, TK = a.I / 16, ncb = TN / NW;
    const int u = blockIdx.x / ncb, cb = blockIdx.x % ncb;    // union entry (or slot with per_slot), column block
    const int blk = HB ? cb >> 1 : cb;                         // its 128-output block
    // one round of independent loads: the union size (slot count), this entry's slot range and its expert's
    // addresses (entries past the count hold stale values and are not used)
    const int U = a.pv.hdr[a.per_slot ? 1 : 0];
    const int s_begin = a.per_slot ? u : a.pv.uoff[u], s_end = a.per_slot ? u + 1 : a.pv.uoff[u + 1];
    const uint8_t* tr = reinterpret_cast<const uint8_t*>(a.pv.uptr[2 * u]);
    const gptr<uint16_t> svh = gaddr<uint16_t>(a.pv.uptr[2 * u + 1]);
    if (u >= U) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, n = lane & 15;
    const int wid = __builtin_amdgcn_readfirstlane(wave);
    const size_t gstride = (size_t)TN * TB;
    const uint8_t* col = tr + (size_t)(cb * NW + wave) * TB;    // this wave's tile column
    const int nbh = a.H / 128;

    const int nsp = NS == 1 ? 1 : max(1, min(NS, a.ns_cap));
    for (int c0 = s_begin; c0 < s_end; c0 += nsp)
    {
        const int ns = NS == 1 ? 1 : min(nsp, s_end - c0);   // >= 1 (c0 < s_end)
        lds_barrier();   // previous pass done with lds_x / lds_y
        // the pass tokens' combine lists (slots in job order and weights): loads issued before the GEMV, written to
        // LDS after it (thread i < ns * topk holds entry i)
        const int ci = threadIdx.x, cs = ci / a.topk, ck = ci % a.topk;
        int q_tok = 0, q_slot = -1, q_npk = 0;
        float q_w = 0.f;
        if (ci < ns * a.topk)
        {
            q_tok = a.pv.slot_pick[c0 + cs] / a.topk;
            q_slot = a.pv.tok_slot[q_tok * a.topk + ck];
            q_w = a.pv.tok_w[q_tok * a.topk + ck];
            q_npk = a.pv.tok_npk[q_tok];
        }
        float res[NS];
        // the pass's down inputs (ns * I fp16) into LDS; each thread's first two 16-byte loads are issued before the
        // trellis groups are requested
        const int nvec = ns * a.I / 8;
        const uint4* xsrc = reinterpret_cast<const uint4*>(a.xtd + (size_t)c0 * a.I);
        // 8 fp16 values -> LDS element 8i.. (widened to fp32 when XF)
        auto put = [&](int i, const uint4& v) {
            if constexpr (XF)
            {
                const uint32_t w[4] = { v.x, v.y, v.z, v.w };
                float4v f0, f1;
#pragma unroll
                for (int q = 0; q < 2; ++q)
                {
                    f0[2 * q] = h2f_bits((uint16_t)w[q]);
                    f0[2 * q + 1] = h2f_bits((uint16_t)(w[q] >> 16));
                    f1[2 * q] = h2f_bits((uint16_t)w[q + 2]);
                    f1[2 * q + 1] = h2f_bits((uint16_t)(w[q + 2] >> 16));
                }
                float4v* d = reinterpret_cast<float4v*>(lds_x) + 2 * i;
                d[0] = f0;
                d[1] = f1;
            }
            else
                reinterpret_cast<uint4*>(lds_x)[i] = v;
        };
        const int i0 = threadIdx.x, i1 = threadIdx.x + NW * 64;
        uint4 xc0 = {}, xc1 = {};
        auto pre_load = [&] {
            if (i0 < nvec) xc0 = xsrc[i0];
            if (i1 < nvec) xc1 = xsrc[i1];
        };
        auto pre = [&] {
            if (i0 < nvec) put(i0, xc0);
            if (i1 < nvec) put(i1, xc1);
            for (int i = threadIdx.x + 2 * NW * 64; i < nvec; i += NW * 64) put(i, xsrc[i]);
            lds_barrier();   // lds_x complete
        };
        if constexpr (MF)
        {
            const float4v acc = chain_mf<K, NGRP>(col, gstride, TK, 0, TK / 8, static_cast<const uint16_t*>(lds_x),
                                                  a.I, ns, rings + wid * RB, pre_load, pre);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
            {
                const int m = 4 * (lane >> 4) + rr;
                if (m < ns) lds_y[m * 128 + wave * 16 + n] = acc[rr];
            }
        }
        else
        {
            chain_dma<K, NS, NGRP, XF>(col, gstride, TK, ns, lds_x, rings + wid * RB, res, pre_load, pre);
            if constexpr (HB)
            {
                // the half block's raw column sums, for whichever half finishes second
                if (lane < 16) st_agent(&a.yd[(size_t)c0 * a.H + cb * (NW * 16) + wave * 16 + n], res[0]);
            }
            else
            {
#pragma unroll
                for (int s = 0; s < NS; ++s)
                    if (s < ns && lane < 16) lds_y[s * 128 + wave * 16 + n] = res[s];
            }
        }
        if (ci < ns * a.topk)
        {
            c_slot[cs][ck] = q_slot;
            c_w[cs][ck] = q_w;
            if (ck == 0) { c_tok[cs] = q_tok; c_npk[cs] = q_npk; }
        }
        if constexpr (HB) release_agent();
        __syncthreads();
        if constexpr (HB)
        {
            // the second half to finish runs out_block (ft_core.h:1016) on the whole 128-block, in place
            if (threadIdx.x == 0)
            {
                int* ctr = a.blk_cnt + ((size_t)c0 * nbh + blk) * CNT_STRIDE;
                const int old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_last[0] = old == 1;
                if (old == 1) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
            if (!s_last[0]) return;
            if (wave == 0)
            {
                float* y = a.yd + (size_t)c0 * a.H + blk * 128;
                float v0 = ld_agent(&y[lane]), v1 = ld_agent(&y[lane + 64]);
                out_block_wave(v0, v1, h2f_bits(svh[blk * 128 + lane]), h2f_bits(svh[blk * 128 + lane + 64]));
                st_agent(&y[lane], v0);
                st_agent(&y[lane + 64], v1);
            }
        }
        else
        {
            // out_block (ft_core.h:1016) of the pass's 128-blocks, published as the experts' outputs
            for (int s = wave; s < ns; s += NW)
            {
                float v0 = lds_y[s * 128 + lane], v1 = lds_y[s * 128 + lane + 64];
                out_block_wave(v0, v1, h2f_bits(svh[blk * 128 + lane]), h2f_bits(svh[blk * 128 + lane + 64]));
                st_agent(&a.yd[(size_t)(c0 + s) * a.H + blk * 128 + lane], v0);
                st_agent(&a.yd[(size_t)(c0 + s) * a.H + blk * 128 + lane + 64], v1);
            }
        }
        release_agent();
        __syncthreads();
        // count this block of every pass token in; the token's last expert sums the block in job order
        if (threadIdx.x < ns)
        {
            const int s = threadIdx.x;
            const int tok = c_tok[s], npk = c_npk[s];
            int* ctr = a.out_cnt + ((size_t)tok * nbh + blk) * CNT_STRIDE;
            const int old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last[s] = old == npk - 1 ? tok : -1;
            if (old == npk - 1) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        for (int s = wave; s < ns; s += NW)
        {
            const int tok = s_last[s];
            if (tok < 0) continue;
            // weighted sum in (job, pick) order (ft_core.h:1020-1033): o = 0, then o += w * y; eight experts' blocks
            // are loaded at a time, unconditionally (past the token's picks its last pick again, never used), so
            // the loads do not wait for one another: one memory round trip at top-8. Then they are added in order.
            const int npk = c_npk[s];
            float o0 = 0.f, o1 = 0.f;
            for (int k0 = 0; k0 < npk; k0 += 8)
            {
                float y0[8], y1[8];
#pragma unroll
                for (int i = 0; i < 8; ++i)
                {
                    const float* y = a.yd + (size_t)c_slot[s][min(k0 + i, npk - 1)] * a.H + blk * 128;
                    y0[i] = ld_agent(&y[lane]);
                    y1[i] = ld_agent(&y[lane + 64]);
                }
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (k0 + i < npk)
                    {
                        o0 = o0 + c_w[s][k0 + i] * y0[i];
                        o1 = o1 + c_w[s][k0 + i] * y1[i];
                    }
            }
            a.out[(size_t)tok * a.H + blk * 128 + lane] = o0;
            a.out[(size_t)tok * a.H + blk * 128 + lane + 64] = o1;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// relay launches: one slot per workgroup (slot = pick), RW waves per tile column
// ---------------------------------------------------------------------------------------------------------------

// LDS of the relay gate|up launch: the waves' rings plus the slot's fp32 inputs, or the plan of the publishing
// workgroup where that is larger
template <int K>
__host__ __device__ constexpr size_t gu_relay_lds(int H, int P, int E)
{
    const size_t x = (size_t)H * 4, plan = lplan_ints(P, E) * 4;
    return (size_t)GU_NW * 8 * 32 * K + (x > plan ? x : plan);
}

// Grid: 8 + relay_blocks(nmat * P * I / (16 * CW)), CW = GU_NW / RW tile columns per workgroup. Item (m * P + p) *
// (I / (16 CW)) + cb: pick p's 16 CW outputs [cb * 16 CW, (cb + 1) * 16 CW) of matrix mat_base + m, RW waves per column
// (chain_relay); a skipped pick's workgroups return at once. Workgroup 0 marks skipped picks for the down launch and
// zeroes the output rows of tokens without a valid pick (slots are picks; the down launch forms each token's combine
// order itself).
// The last of the workgroups covering a 128-block of a pick (gate and up) runs its SwiGLU stage, as in gu_kernel.
template <int K, int RW>
__global__ __launch_bounds__(GU_NW * 64) __attribute__((amdgpu_waves_per_eu(3))) void gu_relay_kernel(GuArgs a)
{
    constexpr int NW = GU_NW, CW = NW / RW, TB = 32 * K;
    static_assert(NW % RW == 0, "relay width divides the workgroup");
    extern __shared__ __align__(16) uint8_t lds_raw[];
    __shared__ int hdr[4];
    __shared__ int s_last;
    __shared__ float relay[CW][64];
    __shared__ int relay_turn[CW];
    if (threadIdx.x < CW) relay_turn[threadIdx.x] = 0;   // ordered before every hand-off by the input barrier
    constexpr int RB = 8 * TB;                                           // one group slot per wave
    uint8_t* rings = lds_raw;                                            // [NW][RB]
    float* lds_x = reinterpret_cast<float*>(lds_raw + NW * RB);          // [H] permuted, fp32
    const int TN = a.I / 16, TK = a.H / 16, ncb = TN / CW;
    if (blockIdx.x == 0)
    {
        relay_plan_block(a.sel, a.P, a.topk, a.E, a.out, a.H, a.pv.uptr, reinterpret_cast<int*>(lds_x));
        return;
    }
    // block 0 marks skipped picks and zeroes the rows of tokens without picks, blocks 1..7 have no work (the items
    // start at an XCD-aligned block); all of them end within a load's latency, so every GEMV workgroup finds a free
    // slot in the first dispatch round
    const int PT = a.P + a.nsh;   // routed picks, then the shared expert's (one per token)
    const long item = blockIdx.x < 8 ? -1 : relay_item(blockIdx.x - 8, RW, (long)a.nmat_launch * PT * ncb);
    if (item < 0) return;
    const int wg = (int)item, per_mat = PT * ncb;
    const int p = (wg % per_mat) / ncb, cb = wg % ncb;
    const int64_t e64 = p < a.P ? a.sel[p] : a.E;   // the shared expert is row E of the table
    if (e64 < 0 || e64 > a.E || (e64 == a.E && p < a.P)) return;
    const int e = (int)e64;
    const int tok = p < a.P ? p / a.topk : p - a.P;
    const int mat = a.mat_base + wg / per_mat;   // 0 gate, 1 up
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, n = lane & 15;
    const int wid = __builtin_amdgcn_readfirstlane(wave);
    const int c = wid / RW, r = wid % RW;
    const uint8_t* tr = reinterpret_cast<const uint8_t*>(a.ptrs[(size_t)e * 9 + mat]);
    const gptr<uint16_t> suh = gaddr<uint16_t>(a.ptrs[(size_t)e * 9 + 3 + 2 * mat]);
    // the pick's down trellis and svh_down addresses for the down launch, from the workgroup of the gate matrix's
    // first column block
    if (mat == 0 && cb == 0 && threadIdx.x < 2) a.pv.uptr[2 * p + threadIdx.x] = a.ptrs[(size_t)e * 9 + 2 + 6 * threadIdx.x];
    const size_t gstride = (size_t)TN * TB;
    const int t = cb * CW + c;   // this wave's tile column
    const uint8_t* col = tr + (size_t)t * TB;
    const uint16_t* xrow = a.x + (size_t)tok * a.H;

    // input transform (prep_block, ft_core.h:97-102) into LDS: each 16-lane row takes one 128-block, 8 elements per
    // lane; the first GU_PR rounds of blocks are loaded before the trellis groups are requested
    const int nblk = TK / 8, rl = lane >> 4, li = lane & 15;
    uint4 xv[GU_PR], sv[GU_PR];
    auto load_round = [&](int rd, int k) {
        const int b = min((rd * NW + wave) * 4 + rl, nblk - 1);
        xv[k] = *reinterpret_cast<const uint4*>(xrow + b * 128 + li * 8);
        sv[k] = gld16(suh, b * 128 + li * 8);
    };
    auto prep_round = [&](int rd, int k) {
        const int b = (rd * NW + wave) * 4 + rl;
        float v[8];
        prep_block_row_p(v, xv[k], sv[k]);
        if (b < nblk)
        {
            // elements 8li..8li+7 of block b: tile row li/2, accumulators j0 = 2(li&1) and j0 + 1, q = k/2
            const int tk = b * 8 + (li >> 1), j0 = 2 * (li & 1);
            float* dst = lds_x + (tk * 4 + j0) * 4;
            float4v e0, e1;
#pragma unroll
            for (int q = 0; q < 4; ++q)
            {
                e0[q] = h2f_bits((uint16_t)f2h_bits(v[2 * q]));
                e1[q] = h2f_bits((uint16_t)f2h_bits(v[2 * q + 1]));
            }
            *reinterpret_cast<float4v*>(dst) = e0;
            *reinterpret_cast<float4v*>(dst + 4) = e1;
        }
    };
    const int nr = (nblk + 4 * NW - 1) / (4 * NW);   // rounds of 4 * NW blocks
    auto pre_load = [&] {
#pragma unroll
        for (int k = 0; k < GU_PR; ++k)
            if (k < nr) load_round(k, k);
    };
    auto pre = [&] {
        for (int r0 = 0; r0 < nr; r0 += GU_PR)
        {
            if (r0 > 0)
            {
#pragma unroll
                for (int k = 0; k < GU_PR; ++k)
                    if (r0 + k < nr) load_round(r0 + k, k);
            }
#pragma unroll
            for (int k = 0; k < GU_PR; ++k)
                if (r0 + k < nr) prep_round(r0 + k, k);
        }
        lds_barrier();   // lds_x complete
    };
    const float res = chain_relay<K, NGRP - 1, RW>(col, gstride, TK, lds_x, rings + wid * RB, relay[c],
                                                   &relay_turn[c], r, a.status, a.spin_max, a.prio, pre_load, pre);
    float* ybase = a.ygu + (size_t)mat * a.pv.cap_slots * a.I;
    if (r == 0 && lane < 16) st_agent(&ybase[(size_t)p * a.I + t * 16 + n], res);
    release_agent();
    __syncthreads();
    const int blk = (cb * CW * 16) / 128;
    if (threadIdx.x == 0)
    {
        int* ctr = a.act_cnt + ((size_t)p * (a.I / 128) + blk) * CNT_STRIDE;
        const int old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == a.nmat_total - 1;
        if (s_last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (s_last) act_block(a, e, p, p + 1, blk);
}

// LDS of the relay down launch: the waves' rings plus the slot's fp32 inputs, or the combining workgroup's blocks of
// up to MAX_TOPK picks and the shared expert's where that is larger
template <int K>
__host__ __device__ constexpr size_t dn_relay_lds(int I)
{
    const size_t x = (size_t)I * 4, comb = (size_t)(MAX_TOPK + 1) * 128 * 4;
    return (size_t)GU_NW * 8 * 32 * K + (x > comb ? x : comb);
}

// Grid: P * H / (16 * CW). Workgroup (p, cb): the raw down sums [cb * 16 CW, (cb + 1) * 16 CW) of pick p (slot p)
// into yd, RW waves per column; the last of the NQ * npk workgroups that cover a token's 128-output block (NQ quarters
// of each of its npk picks) runs out_block on every pick's block and the token's weighted sum of the block, in the
// job order it forms itself from sel (relay_combine_list; wave 0 loads the call's picks, weights and svh_down
// addresses into registers before the GEMV, so none of their latency falls on that tail).
template <int K, int RW>
__global__ __launch_bounds__(GU_NW * 64) __attribute__((amdgpu_waves_per_eu(3))) void dn_relay_kernel(DnArgs a)
{
    constexpr int NW = GU_NW, CW = NW / RW, TB = 32 * K, NQ = 128 / (16 * CW);
    extern __shared__ __align__(16) uint8_t lds_raw[];
    __shared__ int s_last;
    __shared__ int c_npk, c_slot[MAX_TOPK + 1];   // the token's picks in combine order, then its shared-expert pick
    __shared__ float c_w[MAX_TOPK + 1];
    __shared__ uint64_t c_svh[MAX_TOPK + 1];
    __shared__ float relay[CW][64];
    __shared__ int relay_turn[CW];
    if (threadIdx.x < CW) relay_turn[threadIdx.x] = 0;   // ordered before every hand-off by the input barrier
    constexpr int RB = 8 * TB;                                      // one group slot per wave
    uint8_t* rings = lds_raw;                                       // [NW][RB]
    float* lds_x = reinterpret_cast<float*>(lds_raw + NW * RB);     // [I] permuted, fp32
    const int TN = a.H / 16, TK = a.I / 16, ncb = TN / CW;
    const int P = a.pv_picks, PT = P + a.nsh;   // routed picks, then the shared expert's (one per token)
    const long item = relay_item(blockIdx.x, RW, (long)PT * ncb);
    if (item < 0) return;
    const int p = (int)(item / ncb), cb = (int)(item % ncb);
    const int blk = cb / NQ;
    const uint8_t* tr = reinterpret_cast<const uint8_t*>(a.pv.uptr[2 * p]);
    const gptr<uint16_t> svh = gaddr<uint16_t>(a.pv.uptr[2 * p + 1]);
    if (tr == nullptr) return;   // skipped pick
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, n = lane & 15;
    // wave 0: the call's picks, weights and svh_down addresses (lane = pick), for the combine list at the end
    int64_t e_l = -1;
    float w_l = 0.f;
    uint64_t svh_l = 0;
    if (wave == 0 && lane < P)
    {
        e_l = a.sel[lane];
        w_l = a.w_half ? h2f_bits(reinterpret_cast<const uint16_t*>(a.w)[lane]) : reinterpret_cast<const float*>(a.w)[lane];
        svh_l = a.pv.uptr[2 * lane + 1];
    }
    const int wid = __builtin_amdgcn_readfirstlane(wave);
    const int c = wid / RW, r = wid % RW;
    const size_t gstride = (size_t)TN * TB;
    const int t = cb * CW + c;
    const uint8_t* col = tr + (size_t)t * TB;
    const int nbh = a.H / 128;
    const int tok = p < P ? p / a.topk : p - P;
    // the slot's down input (I fp16) into LDS as fp32; each thread's first two 16-byte loads are issued before the
    // trellis groups are requested
    const int nvec = a.I / 8;
    const uint4* xsrc = reinterpret_cast<const uint4*>(a.xtd + (size_t)p * a.I);
    auto put = [&](int i, const uint4& v) {
        const uint32_t w[4] = { v.x, v.y, v.z, v.w };
        float4v f0, f1;
#pragma unroll
        for (int q = 0; q < 2; ++q)
        {
            f0[2 * q] = h2f_bits((uint16_t)w[q]);
            f0[2 * q + 1] = h2f_bits((uint16_t)(w[q] >> 16));
            f1[2 * q] = h2f_bits((uint16_t)w[q + 2]);
            f1[2 * q + 1] = h2f_bits((uint16_t)(w[q + 2] >> 16));
        }
        float4v* d = reinterpret_cast<float4v*>(lds_x) + 2 * i;
        d[0] = f0;
        d[1] = f1;
    };
    const int i0 = threadIdx.x, i1 = threadIdx.x + NW * 64;
    uint4 xc0 = {}, xc1 = {};
    auto pre_load = [&] {
        if (i0 < nvec) xc0 = xsrc[i0];
        if (i1 < nvec) xc1 = xsrc[i1];
    };
    auto pre = [&] {
        if (i0 < nvec) put(i0, xc0);
        if (i1 < nvec) put(i1, xc1);
        for (int i = threadIdx.x + 2 * NW * 64; i < nvec; i += NW * 64) put(i, xsrc[i]);
        lds_barrier();   // lds_x complete
    };
    const float res = chain_relay<K, NGRP - 1, RW>(col, gstride, TK, lds_x, rings + wid * RB, relay[c],
                                                   &relay_turn[c], r, a.status, a.spin_max, a.prio, pre_load, pre);
    if (r == 0 && lane < 16) st_agent(&a.yd[(size_t)p * a.H + t * 16 + n], res);
    // the number of valid picks of the token (its combine's arrival count), from the registers of wave 0
    if (wave == 0)
    {
        const bool mine = lane < P && lane / a.topk == tok && e_l >= 0 && e_l < a.E;
        const uint64_t m = __ballot(mine);
        if (lane == 0) c_npk = __popcll(m);
    }
    release_agent();
    __syncthreads();
    // one counter per (token, 128-block) counts the block's quarter arrivals of every pick of the token; the last
    // arrival runs out_block (ft_core.h:1016) on each pick's block and the weighted sum in (job, pick) order
    // (ft_core.h:1020-1033): o = 0, then o += w * y
    if (threadIdx.x == 0)
    {
        int* ctr = a.out_cnt + ((size_t)tok * nbh + blk) * CNT_STRIDE;
        const int need = NQ * (c_npk + (a.nsh ? 1 : 0));
        const int old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == need - 1;
        if (old == need - 1) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;
    float* ylds = lds_x;   // [npk][128] the picks' blocks after out_block (the GEMV inputs are no longer needed)
    relay_combine_list(e_l, w_l, svh_l, P, a.E, a.topk, tok, c_slot, c_w, c_svh, &c_npk);
    // the shared expert last, weight 1: o + 1 * y = o + y, the join of routed + shared (k_overlap's fp32 add)
    if (a.nsh && threadIdx.x == 0)
    {
        c_slot[c_npk] = P + tok;
        c_w[c_npk] = 1.0f;
        c_svh[c_npk] = a.pv.uptr[2 * (P + tok) + 1];
    }
    __syncthreads();
    const int npk = c_npk + (a.nsh ? 1 : 0);
    // wave w takes picks w, w + NW, ...: every load of its picks is issued before the first out_block, so the wave
    // waits one memory round trip, not one per pick. The loads run unconditionally (past the token's picks on its
    // last pick again, loaded and never used): under a branch each would be waited for before the next was issued.
    constexpr int KPW = (MAX_TOPK + 1 + NW - 1) / NW;
    if (wave < npk)
    {
        float v0[KPW], v1[KPW];
        uint32_t s0[KPW], s1[KPW];
#pragma unroll
        for (int i = 0; i < KPW; ++i)
        {
            const int k = min(wave + i * NW, npk - 1);
            const float* y = a.yd + (size_t)c_slot[k] * a.H + blk * 128;
            const gptr<uint16_t> sv = gaddr<uint16_t>(c_svh[k]);
            v0[i] = ld_agent(&y[lane]);
            v1[i] = ld_agent(&y[lane + 64]);
            s0[i] = sv[blk * 128 + lane];
            s1[i] = sv[blk * 128 + lane + 64];
        }
#pragma unroll
        for (int i = 0; i < KPW; ++i)
        {
            const int k = wave + i * NW;
            if (k < npk)
            {
                out_block_wave(v0[i], v1[i], h2f_bits((uint16_t)s0[i]), h2f_bits((uint16_t)s1[i]));
                ylds[k * 128 + lane] = v0[i];
                ylds[k * 128 + lane + 64] = v1[i];
            }
        }
    }
    __syncthreads();
    if (wave != 0) return;
    float o0 = 0.f, o1 = 0.f;
    for (int k = 0; k < npk; ++k)
    {
        o0 = o0 + c_w[k] * ylds[k * 128 + lane];
        o1 = o1 + c_w[k] * ylds[k * 128 + lane + 64];
    }
    a.out[(size_t)tok * a.H + blk * 128 + lane] = o0;
    a.out[(size_t)tok * a.H + blk * 128 + lane + 64] = o1;
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

// Every kernel with dynamic LDS is opened once per process (thread-safe static initialisation) to the 160 KB of a
// workgroup minus its own static LDS; the launch itself asks for what it needs. Returns false when the runtime refuses.
template <typename F>
static bool open_lds(F kern)
{
    hipFuncAttributes at;
    if (hipFuncGetAttributes(&at, reinterpret_cast<const void*>(kern)) != hipSuccess) return false;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               LDS_LIMIT - (int)at.sharedSizeBytes) == hipSuccess;
}

// gplan: the plan comes from pv (plan_kernel), so none is built in LDS
template <int K>
static size_t gu_lds(int ns, int H, int P, int E, int mf, int gplan)
{
    return (size_t)GU_NW * NGRP * 8 * 32 * K + (size_t)ns * H * (mf ? 1 : x_lds_elem(ns)) +
           (gplan ? 0 : lplan_ints(P, E) * 4);
}

template <int K>
static size_t dn_lds(int ns, int I, int mf)
{
    const int nw = (ns == 1 && !mf) ? DN_NW / 2 : DN_NW;
    return (size_t)nw * NGRP * 8 * 32 * K + (size_t)ns * I * (mf ? 2 : x_lds_elem(ns)) + (size_t)ns * 128 * 4;
}

template <int K, int NS, bool MF>
static void gu_launch(const GuArgs& a, int umax, int nmat, hipStream_t st)
{
    const size_t lds = gu_lds<K>(a.ns_cap, a.H, a.P, a.E, MF, a.gplan);
    auto kern = gu_kernel<K, NS, MF>;
    static const bool opened = open_lds(kern);
    (void)opened;
    const int ents = a.per_slot ? a.P : umax;
    const int per_ent = (a.I / (16 * GU_NW)) * (MF ? 2 : 1);   // MF: both halves of the tile rows
    timed_launch(kern, dim3(ents * per_ent + 1, nmat), dim3(GU_NW * 64), lds, st, a);
}

static void plan_launch(const GuArgs& a, hipStream_t st)
{
    static const bool opened = open_lds(plan_kernel);
    (void)opened;
    timed_launch(plan_kernel, dim3(1), dim3(GU_NW * 64), (lplan_ints(a.P, a.E) + a.P) * 4, st, a);
}

template <int K, int NS, bool MF>
static void dn_launch(const DnArgs& a, int umax, int P, hipStream_t st)
{
    const size_t lds = dn_lds<K>(a.ns_cap, a.I, MF);
    auto kern = down_kernel<K, NS, MF>;
    static const bool opened = open_lds(kern);
    (void)opened;
    const int ents = a.per_slot ? P : umax;
    constexpr int nw = (NS == 1 && !MF) ? DN_NW / 2 : DN_NW;
    timed_launch(kern, dim3(ents * (a.H / (16 * nw))), dim3(nw * 64), lds, st, a);
}

// Compute units of the current device (cached per device).
static int device_cus()
{
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev])
    {
        int n = 0;
        cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n
                                                                                                              : 256;
    }
    return cus[dev];
}

// LDS to request for a launch of nwg equal workgroups that each need `need` bytes: at least enough that a CU holds
// no more than ceil(nwg / CUs) of them. The relay kernels use few registers, so the dispatcher could otherwise put one
// workgroup more on some CUs than on the rest, and those CUs set the launch's time.
static size_t balanced_lds(size_t need, long nwg)
{
    const long cus = device_cus(), per_cu = (nwg + cus - 1) / cus;
    const size_t cap = (size_t)LDS_LIMIT / (size_t)(per_cu + 1) + 16;
    return cap > need && cap <= (size_t)LDS_LIMIT ? cap : need;
}

// Waves of a kernel that one SIMD holds at once, from its register count (512 VGPRs per lane, allocated in blocks of
// 8; at most 8 waves).
static int resident_waves(const void* kern)
{
    hipFuncAttributes at{};
    if (hipFuncGetAttributes(&at, kern) != hipSuccess || at.numRegs <= 0) return 3;
    const int regs = (at.numRegs + 7) / 8 * 8;
    return std::min(8, 512 / regs);
}

// Progress priority of a relay launch (chain_relay's prio): on when the launch puts more than one wave on a SIMD and
// all of them fit at once (cap: resident_waves), so that a SIMD's last wave would otherwise run its last stretch
// alone. Measured on MI355X (config 1, us per token): M = 1 (gate|up 3 waves per SIMD of 3, down 2.5 of 4) 48.9 ->
// 45.8; M = 2 with it on gate|up (3 of 4) 36.6 -> 34.9, while on down as well (5 waves per SIMD, two rounds) 0.4
// slower; routed + shared expert in one call at M = 2 (gate|up 3.4 of 4) 42.4 -> 40.0. prio >= 0 (GFL_RELAY_PRIO)
// forces it.
static int relay_prio(int prio, long waves, int cap)
{
    if (prio >= 0) return prio;
    const long simds = 4L * device_cus();
    return waves > simds && waves <= cap * simds ? 1 : 0;
}

template <int K, int RW>
static void gu_relay_launch(const GuArgs& a, int nmat, hipStream_t st)
{
    constexpr int CW = GU_NW / RW;
    auto kern = gu_relay_kernel<K, RW>;
    static const bool opened = open_lds(kern);
    (void)opened;
    const long nwg = (long)(a.P + a.nsh) * (a.I / (16 * CW)) * nmat;   // GEMV workgroups (plus the publishing one)
    const size_t lds = balanced_lds(gu_relay_lds<K>(a.H, a.P, a.E), nwg);
    GuArgs b = a;
    b.nmat_launch = nmat;
    static const int cap = resident_waves(reinterpret_cast<const void*>(kern));
    b.prio = relay_prio(a.prio, nwg * GU_NW, cap);
    timed_launch(kern, dim3(8 + relay_blocks(nwg, RW)), dim3(GU_NW * 64), lds, st, b);
}

template <int K, int RW>
static void dn_relay_launch(const DnArgs& a, int P, hipStream_t st)
{
    constexpr int CW = GU_NW / RW;
    auto kern = dn_relay_kernel<K, RW>;
    static const bool opened = open_lds(kern);
    (void)opened;
    const long nwg = (long)(P + a.nsh) * (a.H / (16 * CW));
    const size_t lds = balanced_lds(dn_relay_lds<K>(a.I), nwg);
    DnArgs b = a;
    b.pv_picks = P;
    static const int cap = resident_waves(reinterpret_cast<const void*>(kern));
    b.prio = relay_prio(a.prio, nwg * GU_NW, cap);
    timed_launch(kern, dim3(relay_blocks(nwg, RW)), dim3(GU_NW * 64), lds, st, b);
}

// relay width: 1, 2 or 4 waves per tile column
#define GFL_RW_SWITCH(RWV, CALL)                                                                                \
    if ((RWV) == 1) { constexpr int RW_ = 1; CALL; }                                                           \
    else if ((RWV) == 2) { constexpr int RW_ = 2; CALL; }                                                      \
    else { constexpr int RW_ = 4; CALL; }

// slots per pass: 1, 4 or 8 (a 2-slot instantiation does not fit the register budget without spilling; passes with
// fewer slots than NS skip the unused ones)
#define GFL_NS_SWITCH(NSV, CALL)                                                                                \
    if ((NSV) <= 1) { constexpr int NS_ = 1; CALL; }                                                           \
    else if ((NSV) <= 4) { constexpr int NS_ = 4; CALL; }                                                      \
    else { constexpr int NS_ = 8; CALL; }

#define GFL_K_SWITCH(KV, CALL)                                                                                  \
    switch (KV)                                                                                                 \
    {                                                                                                           \
        case 2: { constexpr int K_ = 2; CALL; } break;                                                          \
        case 3: { constexpr int K_ = 3; CALL; } break;                                                          \
        case 4: { constexpr int K_ = 4; CALL; } break;                                                          \
        case 5: { constexpr int K_ = 5; CALL; } break;                                                          \
        default: return -1;                                                                                     \
    }

size_t gate_up_lds_bytes(int K, int ns, int H, int P, int E, int mf, int rw, int gplan)
{
    size_t r = 0;
    auto f = [&]() -> int {
        GFL_K_SWITCH(K, (r = rw ? gu_relay_lds<K_>(H, P, E) : gu_lds<K_>(ns, H, P, E, mf, gplan)))
        return 0;
    };
    f();
    return r;
}

size_t down_lds_bytes(int K, int ns, int I, int P, int E, int mf, int rw)
{
    size_t r = 0;
    auto f = [&]() -> int {
        GFL_K_SWITCH(K, (r = rw ? dn_relay_lds<K_>(I) : dn_lds<K_>(ns, I, mf)))
        return 0;
    };
    f();
    return r;
}

int launch_gate_up(int K, int ns, const uint64_t* ptrs, int mat_base, int nmat, const int64_t* sel, const void* w,
                   int w_half, int P, int topk, int E, int H, int I, int umax, const uint16_t* x, float* ygu,
                   uint16_t* xtd, int* act_cnt, const float* silu_tab, float act_limit, const PlanView& pv, float* out,
                   int mf, int rw, int prio, int nsh, int gplan, int* status, int spin_max, hipStream_t st)
{
    if (nsh && (!rw || mf)) return -1;   // shared-expert picks ride on the relay launches only
    GuArgs a;
    a.status = status; a.spin_max = spin_max; a.nmat_launch = nmat; a.gplan = rw ? 0 : gplan;
    a.prio = rw ? prio : 0;
    a.nsh = nsh;
    a.ptrs = ptrs; a.sel = sel; a.w = w; a.w_half = w_half; a.P = P; a.topk = topk; a.E = E; a.H = H; a.I = I;
    a.mat_base = mat_base; a.x = x; a.ygu = ygu; a.xtd = xtd; a.act_cnt = act_cnt; a.silu_tab = silu_tab;
    a.act_limit = act_limit; a.pv = pv; a.out = out;
    a.ns_cap = ns;
    a.mf = mf;
    if (mf)
    {
        // MFMA-accumulate mode: workgroups per union entry, all its slots in passes of up to ns
        a.nmat_total = 2 * 2 * (128 / (16 * GU_NW));   // gate, up x two halves
        a.per_slot = 0;
        if (a.gplan && mat_base == 0) plan_launch(a, st);
        GFL_K_SWITCH(K, (gu_launch<K_, 4, true>(a, umax, nmat, st)))
        return 0;
    }
    if (rw)
    {
        // one slot per workgroup, slot = pick, rw waves per tile column
        a.nmat_total = 2 * (128 / (16 * (GU_NW / rw)));
        a.per_slot = 1;
        GFL_K_SWITCH(K, GFL_RW_SWITCH(rw, (gu_relay_launch<K_, RW_>(a, nmat, st))))
        return 0;
    }
    a.nmat_total = 2 * (128 / (16 * GU_NW));
    a.per_slot = ns == 1;
    if (a.gplan && mat_base == 0) plan_launch(a, st);
    GFL_K_SWITCH(K, GFL_NS_SWITCH(ns, (gu_launch<K_, NS_, false>(a, umax, nmat, st))))
    return 0;
}

int launch_down(int K, int ns, const uint64_t* ptrs, int topk, int H, int I, int umax, int P, int E, const int64_t* sel,
                const void* w, int w_half, const PlanView& pv, const uint16_t* xtd, float* yd, int* out_cnt,
                int* blk_cnt, float* out, int mf, int rw, int prio, int nsh, int* status, int spin_max,
                hipStream_t st)
{
    if (nsh && (!rw || mf)) return -1;
    DnArgs a;
    a.status = status; a.spin_max = spin_max; a.pv_picks = P;
    a.prio = rw ? prio : 0;
    a.nsh = nsh;
    a.sel = sel; a.w = w; a.w_half = w_half; a.E = E;
    a.ptrs = ptrs; a.topk = topk; a.H = H; a.I = I; a.pv = pv; a.xtd = xtd; a.yd = yd; a.out_cnt = out_cnt;
    a.blk_cnt = blk_cnt;
    a.out = out;
    a.ns_cap = ns;
    if (mf)
    {
        a.per_slot = 0;
        GFL_K_SWITCH(K, (dn_launch<K_, 4, true>(a, umax, P, st)))
        return 0;
    }
    if (rw)
    {
        // relay_combine_list holds the call's picks one per lane of a wave
        if (P > 64) return -1;
        a.per_slot = 1;
        GFL_K_SWITCH(K, GFL_RW_SWITCH(rw, (dn_relay_launch<K_, RW_>(a, P, st))))
        return 0;
    }
    a.per_slot = ns == 1;
    GFL_K_SWITCH(K, GFL_NS_SWITCH(ns, (dn_launch<K_, NS_, false>(a, umax, P, st))))
    return 0;
}
#undef GFL_NS_SWITCH
#undef GFL_RW_SWITCH
#undef GFL_K_SWITCH

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
