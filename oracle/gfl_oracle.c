/* CPU oracle for the routed-MoE expert path -- TEST INFRASTRUCTURE ONLY (see gfl_oracle.h).
 *
 * Built with -ffp-contract=off so every multiply-add below is rounded exactly where the source says: explicit
 * fmaf() where the reference uses an FMA intrinsic, separate mul/add everywhere else. This is what makes the EXACT
 * path bit-identical to the reference's own EXACT mode compiled with -ffp-contract=off.
 *
 * Parity status (checked by tests/test_oracle.py):
 *   decode/dequant K=3   pinned: golden vectors from the reference's dense_weights + a naive bit-string decoder
 *   decode K=4,5         pinned: naive bit-string decoder + low-K-bits invariant (no reference K=4/5 decode exists)
 *   transforms/EXACT     pinned: golden vectors from the reference's moe_forward(EXACT) and ref_expert
 *   AFFINE               pinned: golden vectors from the reference's moe_forward(AFFINE)
 *   split                pinned: identity/stats invariants, brute-force cost-model argmin, fast==stock order rules
 *   grouped rows, router pinned: brute-force sort-based construction; router closed form (exllamav3 router itself
 *                        is not in the reference tree: parity unpinned against exllamav3)
 */
#include "gfl_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define MUL1 0x83DCD12Du
#define HAD 0.088388347648f

/* ------------------------------------------------------------------------------------------------------------ */
/* fp16                                                                                                          */
/* ------------------------------------------------------------------------------------------------------------ */

float gflo_h2f(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t x;
    if (e == 0)
    {
        if (m == 0) x = sign;
        else
        {
            /* subnormal half: m * 2^-24 */
            float f = (float)m * 5.9604644775390625e-8f;
            memcpy(&x, &f, 4);
            x |= sign;
        }
    }
    else if (e == 31) x = sign | 0x7F800000u | (m << 13);
    else x = sign | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &x, 4);
    return f;
}

uint16_t gflo_f2h(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return sign | (a > 0x7F800000u ? 0x7E00u : 0x7C00u);
    if (a >= 0x477FF000u) return sign | 0x7C00u;                 /* rounds to infinity */
    if (a < 0x38800000u)
    {
        /* half subnormal: value in units of 2^-24, round to nearest even */
        const int e = (int)(a >> 23);
        if (e < 102) return sign;
        const uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
        const int sh = 126 - e;
        uint32_t r = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return sign | (uint16_t)r;
    }
    const uint32_t r = a - 0x38000000u;
    uint32_t h = r >> 13;
    const uint32_t rem = r & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return sign | (uint16_t)h;
}

float gflo_r16(float f) { return gflo_h2f(gflo_f2h(f)); }

/* ------------------------------------------------------------------------------------------------------------ */
/* format                                                                                                        */
/* ------------------------------------------------------------------------------------------------------------ */

static uint32_t ld32(const uint16_t* p, int i)
{
    uint32_t v;
    memcpy(&v, p + i * 2, 4);
    return v;
}

/* state_scalar (ft_core.h:65-73) with BITS generalised to K: the tile is a circular 256*K-bit stream, MSB-first
 * inside little-endian 32-bit words; state t is the 16 bits ending at bit (t+1)*K. */
uint16_t gflo_state(const uint16_t* packed, int K, int t)
{
    const int words32 = K * 256 / 32;
    const int b0 = t * K + K - 16 + 256 * K;
    const int b1 = b0 + 16;
    const int shift = ((b1 - 1) / 32 + 1) * 32 - b1;
    const uint64_t merged = ((uint64_t)ld32(packed, (b0 / 32) % words32) << 32) | ld32(packed, ((b1 - 1) / 32) % words32);
    return (uint16_t)(merged >> shift);
}

/* init_perm (ft_core.h:50-61) */
int gflo_perm(int i)
{
    const int t = i / 8, j = i % 8;
    const int r0 = (t % 4) * 2;
    const int rows[4] = { r0, r0 + 1, r0 + 8, r0 + 9 };
    const int c = t / 4 + (j >= 4 ? 8 : 0);
    return rows[j % 4] * 16 + c;
}

int gflo_bytesum(uint16_t st)
{
    const uint32_t x = (uint32_t)st * MUL1;
    return (int)((x & 0xffu) + ((x >> 8) & 0xffu) + ((x >> 16) & 0xffu) + (x >> 24));
}

static float kinv(void) { return gflo_h2f(0x1eee); }
static float kbias(void) { return gflo_h2f(0xc931); }
static float caff(void) { return 1024.0f * gflo_h2f(0x1eee) + gflo_h2f(0xc931); }   /* exact in fp32 */

/* w_gpu (ft_core.h:82): one fp16 rounding of an exact fp32 fma */
uint16_t gflo_weight_bits(uint16_t st)
{
    return gflo_f2h(fmaf((float)(1024 + gflo_bytesum(st)), kinv(), kbias()));
}

/* dense_weights (ft_core.h:1657-1672) */
void gflo_dequant(const uint8_t* tr, int k, int n, int K, uint16_t* W)
{
    const int tn = n / 16, tb = 32 * K;
    for (int tk = 0; tk < k / 16; ++tk)
        for (int t = 0; t < tn; ++t)
        {
            const uint16_t* packed = (const uint16_t*)(tr + ((size_t)tk * tn + t) * tb);
            for (int i = 0; i < 256; ++i)
            {
                const int rc = gflo_perm(i);
                W[(size_t)(tk * 16 + rc / 16) * n + t * 16 + rc % 16] = gflo_weight_bits(gflo_state(packed, K, i));
            }
        }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* transforms                                                                                                    */
/* ------------------------------------------------------------------------------------------------------------ */

/* had128 (ft_core.h:89-94): natural-order Sylvester butterflies */
void gflo_had128(float* v)
{
    for (int w = 1; w < 128; w *= 2)
        for (int b = 0; b < 128; b += 2 * w)
            for (int i = 0; i < w; ++i)
            {
                const float a = v[b + i], c = v[b + w + i];
                v[b + i] = a + c;
                v[b + w + i] = a - c;
            }
}

/* prep_block (ft_core.h:97-102) */
void gflo_prep_block(const float* x, const uint16_t* suh, float* xt)
{
    for (int i = 0; i < 128; ++i) xt[i] = x[i] * gflo_h2f(suh[i]);
    gflo_had128(xt);
    for (int i = 0; i < 128; ++i) xt[i] = gflo_r16(xt[i] * HAD);
}

/* out_block (ft_core.h:105-110) */
void gflo_out_block(float* y, const uint16_t* svh)
{
    for (int i = 0; i < 128; ++i) y[i] = gflo_r16(y[i]);
    gflo_had128(y);
    for (int i = 0; i < 128; ++i) y[i] = gflo_r16(y[i] * HAD * gflo_h2f(svh[i]));
}

/* silu + act_mul with the exllamav3 clamp semantics (ft_core.h:123-132); limit 0 = off */
float gflo_act_mul(float g, float u, float limit)
{
    float x = g / (1.0f + expf(-g));
    if (limit != 0.0f)
    {
        u = fminf(fmaxf(u, -limit), limit);
        x = fminf(x, limit);
    }
    return x * u;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* GEMV                                                                                                          */
/* ------------------------------------------------------------------------------------------------------------ */

/* EXACT: per (tile column t, in-tile column c, lane j) one fp32 accumulator, FMA over tile rows then over the four
 * stream groups q of the tile (tile_accum<M,EXACT>, ft_core.h:313-345); lanes reduced (v0+v1)+(v2+v3)
 * (gemv_block, ft_core.h:377-386). AFFINE: the same chain over the raw byte sums, then KINV*lo + CAFF*sum(x). */
/* the GEMV's weight of every 16-bit state, tabulated once from the functions above: EXACT r16(fma(bytesum, KINV,
 * CAFF)) (= the fp16 weight, w_gpu, ft_core.h:82) and the raw byte sum for AFFINE */
static float g_wt_exact[65536], g_wt_sum[65536];
static int g_wt_ready;

static void weight_tables(void)
{
    if (g_wt_ready) return;
    const float KI = kinv(), CA = caff();
    for (uint32_t st = 0; st < 65536; ++st)
    {
        const int bs = gflo_bytesum((uint16_t)st);
        g_wt_exact[st] = gflo_r16(fmaf((float)bs, KI, CA));
        g_wt_sum[st] = (float)bs;
    }
    g_wt_ready = 1;
}

void gflo_gemv(const uint8_t* tr, int k, int n, int K, const float* xt, int M, float* y, int mode,
               const float* sumx_in)
{
    weight_tables();
    const float* wtab = mode == 1 ? g_wt_exact : g_wt_sum;
    const int tn = n / 16, tkn = k / 16, tb = 32 * K;
    const float KI = kinv(), CA = caff();
    float* wt = (float*)malloc(sizeof(float) * 256);
    float* sumx = (float*)calloc((size_t)(M > 0 ? M : 1), sizeof(float));
    float (*acc)[8][8] = (float (*)[8][8])malloc(sizeof(float) * 64 * (size_t)(M > 0 ? M : 1));
    /* each token's chains are independent: a tile is decoded once and fed to every token's accumulators in turn */
    for (int i = 0; i < M; ++i)
    {
        const float* xi = xt + (size_t)i * k;
        if (mode == 0 && sumx_in) sumx[i] = sumx_in[i];
        else if (mode == 0)
            for (int r = 0; r < k; ++r) sumx[i] += xi[r];
    }
    for (int t = 0; t < tn; ++t)
    {
        memset(acc, 0, sizeof(float) * 64 * (size_t)M);
        for (int tk = 0; tk < tkn; ++tk)
        {
            const uint16_t* packed = (const uint16_t*)(tr + ((size_t)tk * tn + t) * tb);
            for (int s = 0; s < 256; ++s) wt[s] = wtab[gflo_state(packed, K, s)];
            for (int i = 0; i < M; ++i)
            {
                const float* xi = xt + (size_t)i * k;
                for (int c = 0; c < 8; ++c)
                    for (int q = 0; q < 4; ++q)
                    {
                        const int g = 4 * c + q, r0 = 2 * q;
                        const int rows[4] = { r0, r0 + 1, r0 + 8, r0 + 9 };
                        for (int j = 0; j < 8; ++j)
                            acc[i][c][j] = fmaf(wt[8 * g + j], xi[tk * 16 + rows[j % 4]], acc[i][c][j]);
                    }
            }
        }
        for (int i = 0; i < M; ++i)
            for (int c = 0; c < 8; ++c)
            {
                const float* v = acc[i][c];
                float lo = (v[0] + v[1]) + (v[2] + v[3]), hi = (v[4] + v[5]) + (v[6] + v[7]);
                if (mode == 0)
                {
                    lo = KI * lo + CA * sumx[i];
                    hi = KI * hi + CA * sumx[i];
                }
                y[(size_t)i * n + t * 16 + c] = lo;
                y[(size_t)i * n + t * 16 + c + 8] = hi;
            }
    }
    free(acc);
    free(sumx);
    free(wt);
}

/* prep of a whole vector, returning sum(xt) accumulated block by block in element order (fwd_phase phase 0) */
static float prep_vector(const float* x, const uint16_t* suh, int k, float* xt)
{
    float s = 0.0f;
    for (int b = 0; b < k / 128; ++b)
    {
        gflo_prep_block(x + b * 128, suh + b * 128, xt + b * 128);
        for (int r = 0; r < 128; ++r) s += xt[b * 128 + r];
    }
    return s;
}

/* fwd_phase phases 0-2 for one expert (ft_core.h:933-1019); the AFFINE sums are re-derived per GEMV, which is
 * the same float sequence as the reference's phase-0 / per-block sums. */
void gflo_expert_forward(const gflo_expert* E, const float* x, int M, float* y, int mode, float act_limit)
{
    const int H = E->g.k, I = E->g.n;
    float* xg = (float*)malloc(sizeof(float) * (size_t)M * H);
    float* xu = (float*)malloc(sizeof(float) * (size_t)M * H);
    float* yg = (float*)malloc(sizeof(float) * (size_t)M * I);
    float* yu = (float*)malloc(sizeof(float) * (size_t)M * I);
    float* xd = (float*)malloc(sizeof(float) * (size_t)M * I);
    for (int i = 0; i < M; ++i)
    {
        prep_vector(x + (size_t)i * H, E->g.suh, H, xg + (size_t)i * H);
        prep_vector(x + (size_t)i * H, E->u.suh, H, xu + (size_t)i * H);
    }
    gflo_gemv(E->g.tr, H, I, E->g.K, xg, M, yg, mode, NULL);
    gflo_gemv(E->u.tr, H, I, E->u.K, xu, M, yu, mode, NULL);
    float* sd = (float*)calloc((size_t)M, sizeof(float));
    for (int i = 0; i < M; ++i)
        for (int b = 0; b < I / 128; ++b)
        {
            float* g = yg + (size_t)i * I + b * 128;
            float* u = yu + (size_t)i * I + b * 128;
            gflo_out_block(g, E->g.svh + b * 128);
            gflo_out_block(u, E->u.svh + b * 128);
            float a[128];
            for (int r = 0; r < 128; ++r) a[r] = gflo_r16(gflo_act_mul(g[r], u[r], act_limit));
            gflo_prep_block(a, E->d.suh + b * 128, xd + (size_t)i * I + b * 128);
            float s = 0.0f;
            for (int r = 0; r < 128; ++r) s += xd[(size_t)i * I + b * 128 + r];
            sd[i] += s;
        }
    gflo_gemv(E->d.tr, I, H, E->d.K, xd, M, y, mode, sd);
    free(sd);
    for (int i = 0; i < M; ++i)
        for (int b = 0; b < H / 128; ++b) gflo_out_block(y + (size_t)i * H + b * 128, E->d.svh + b * 128);
    free(xg); free(xu); free(yg); free(yu); free(xd);
}

/* ref_linear / ref_expert (ft_core.h:1674-1691): fp64 accumulation over the exact fp16 weights */
static void ref_linear(const gflo_mat* m, const float* x, float* y)
{
    float* xt = (float*)malloc(sizeof(float) * m->k);
    uint16_t* W = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)m->k * m->n);
    double* acc = (double*)calloc(m->n, sizeof(double));
    for (int b = 0; b < m->k / 128; ++b) gflo_prep_block(x + b * 128, m->suh + b * 128, xt + b * 128);
    gflo_dequant(m->tr, m->k, m->n, m->K, W);
    for (int k = 0; k < m->k; ++k)
    {
        const double xv = xt[k];
        const uint16_t* wr = W + (size_t)k * m->n;
        for (int n = 0; n < m->n; ++n) acc[n] += xv * (double)gflo_h2f(wr[n]);
    }
    for (int n = 0; n < m->n; ++n) y[n] = (float)acc[n];
    for (int b = 0; b < m->n / 128; ++b) gflo_out_block(y + b * 128, m->svh + b * 128);
    free(xt); free(W); free(acc);
}

void gflo_expert_ref64(const gflo_expert* E, const float* x, float* y, float act_limit)
{
    const int I = E->g.n;
    float* g = (float*)malloc(sizeof(float) * I);
    float* u = (float*)malloc(sizeof(float) * I);
    float* a = (float*)malloc(sizeof(float) * I);
    ref_linear(&E->g, x, g);
    ref_linear(&E->u, x, u);
    for (int i = 0; i < I; ++i) a[i] = gflo_r16(gflo_act_mul(g[i], u[i], act_limit));
    ref_linear(&E->d, a, y);
    free(g); free(u); free(a);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* MoE layer                                                                                                     */
/* ------------------------------------------------------------------------------------------------------------ */

/* job build (ft_core.h:1343-1349): token-major scan, one job per expert in first-appearance order, a new job when
 * the expert's job already holds 8 tokens */
int gflo_build_jobs(int E, int ntok, const int32_t* sel, const float* w, int topk, int32_t* job_e, int32_t* job_m,
                    int32_t* job_tok, float* job_w)
{
    int32_t* jid = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    for (int e = 0; e < E; ++e) jid[e] = -1;
    int nj = 0;
    for (int t = 0; t < ntok; ++t)
        for (int j = 0; j < topk; ++j)
        {
            const int e = sel[t * topk + j];
            if (e < 0) continue;
            if (jid[e] < 0 || job_m[jid[e]] == 8)
            {
                jid[e] = nj;
                job_e[nj] = e;
                job_m[nj] = 0;
                ++nj;
            }
            const int J = jid[e];
            job_tok[J * 8 + job_m[J]] = t;
            job_w[J * 8 + job_m[J]] = w[t * topk + j];
            ++job_m[J];
        }
    free(jid);
    return nj;
}

int gflo_moe_forward_rows(const gflo_expert* experts, int E, const float* x, int ntok, const int32_t* sel,
                          const float* w, int topk, const uint8_t* want, float* out, int mode, float act_limit)
{
    const int H = experts[0].g.k;
    const int cap = ntok * topk;
    int32_t* je = (int32_t*)malloc(sizeof(int32_t) * (size_t)(cap + 1));
    int32_t* jm = (int32_t*)malloc(sizeof(int32_t) * (size_t)(cap + 1));
    int32_t* jt = (int32_t*)malloc(sizeof(int32_t) * (size_t)(cap + 1) * 8);
    float* jw = (float*)malloc(sizeof(float) * (size_t)(cap + 1) * 8);
    const int nj = gflo_build_jobs(E, ntok, sel, w, topk, je, jm, jt, jw);
    float* yd = (float*)malloc(sizeof(float) * (size_t)(nj + 1) * 8 * H);
    float* xj = (float*)malloc(sizeof(float) * (size_t)8 * H);
    float* yj = (float*)malloc(sizeof(float) * (size_t)8 * H);
    int mem[8];
    for (int j = 0; j < nj; ++j)
    {
        /* the job's members (all, or those whose rows are wanted); each token's expert output depends on its own
           input only, so a job may be evaluated for a subset of its members */
        int m = 0;
        for (int i = 0; i < jm[j]; ++i)
            if (!want || want[jt[j * 8 + i]]) mem[m++] = i;
        if (m == 0) continue;
        for (int q = 0; q < m; ++q)
            memcpy(xj + (size_t)q * H, x + (size_t)jt[j * 8 + mem[q]] * H, sizeof(float) * H);
        gflo_expert_forward(&experts[je[j]], xj, m, yj, mode, act_limit);
        for (int q = 0; q < m; ++q)
            memcpy(yd + ((size_t)j * 8 + mem[q]) * H, yj + (size_t)q * H, sizeof(float) * H);
    }
    /* weighted accumulate in job order (fwd_phase phase 3, ft_core.h:1020-1033) */
    memset(out, 0, sizeof(float) * (size_t)ntok * H);
    for (int t = 0; t < ntok; ++t)
    {
        if (want && !want[t]) continue;
        for (int j = 0; j < nj; ++j)
            for (int i = 0; i < jm[j]; ++i)
                if (jt[j * 8 + i] == t)
                {
                    const float* y = yd + ((size_t)j * 8 + i) * H;
                    const float wt = jw[j * 8 + i];
                    float* o = out + (size_t)t * H;
                    for (int c = 0; c < H; ++c) o[c] += wt * y[c];
                }
    }
    free(je); free(jm); free(jt); free(jw); free(yd); free(xj); free(yj);
    return nj;
}

int gflo_moe_forward(const gflo_expert* experts, int E, const float* x, int ntok, const int32_t* sel,
                     const float* w, int topk, float* out, int mode, float act_limit)
{
    return gflo_moe_forward_rows(experts, E, x, ntok, sel, w, topk, NULL, out, mode, act_limit);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* split / combine                                                                                               */
/* ------------------------------------------------------------------------------------------------------------ */

static int h_nonzero(uint16_t h) { return (h & 0x7FFFu) != 0; }

/* ft_split_k thread-0 semantics (ft_tier_cu.cu:53-156); ft_split_fast_k produces the same outputs
 * (ft_split_fast.cu:1-10). Float expressions are evaluated uncontracted, in source order. */
void gflo_split(const int64_t* sel, const uint16_t* w, const uint16_t* z, int n, int bsz, int topk, int H, int E,
                int first, const int32_t* slotof, const float* score, const float* p, int64_t* ctrl, uint16_t* hx,
                int32_t* hpicks, int64_t seq, int li, int keep_ids, int64_t* sel_out, uint16_t* w_out,
                int64_t* dflag, int64_t* stats, const int32_t* rres)
{
    int* cnt = (int*)calloc((size_t)E + 1, sizeof(int));
    unsigned char* cpu = (unsigned char*)calloc((size_t)E + 1, 1);
    int* miss = (int*)malloc(sizeof(int) * ((size_t)E + 1));
    int* rmiss = (int*)malloc(sizeof(int) * ((size_t)E + 1));
    for (int s = 0; s < n; ++s)
    {
        const int64_t e = sel[s] - first;
        if (h_nonzero(w[s]) && e >= 0 && e < E) ++cnt[e];
    }
    int nm = 0, nh = 0, nr = 0;
    const int tri = p[8] > 0.5f && rres != NULL && (int)p[6] < 0;
    const int lut = p[12] > 0.0f;
    for (int e = 0; e < E; ++e)
    {
        if (!cnt[e]) continue;
        if (slotof[e] >= 0) { ++nh; continue; }
        int* l = (tri && rres[e]) ? rmiss : miss;
        int b = (l == rmiss) ? nr++ : nm++;
        while (b > 0 && score[l[b - 1]] > score[e]) { l[b] = l[b - 1]; --b; }
        l[b] = e;
    }
    int best = 0, bestr = 0;
    const int force = (int)p[6];
    const int maxc = (int)p[5] < nm ? (int)p[5] : nm;
    if (force >= 0) best = force < nm ? force : nm;
    else if (tri)
    {
        float bt = 1e30f, cr = 0.0f;
        for (int kr = 0; kr <= nr; ++kr)
        {
            if (kr) { const float f = p[4] * (float)(cnt[rmiss[kr - 1]] - 1); const float g = 1.0f + f; const float h = p[10] * g; cr = cr + h; }
            const float rem = kr ? p[9] + cr : 0.0f;
            float c = 0.0f, cx = 0.0f;
            for (int k = 0; k <= maxc; ++k)
            {
                if (k)
                {
                    const float f = p[4] * (float)(cnt[miss[k - 1]] - 1); const float g = 1.0f + f; const float h = p[3] * g;
                    c = c + h;
                    const float f2 = p[3] * p[4]; const float h2 = f2 * (float)(cnt[miss[k - 1]] - 1);
                    cx = cx + h2;
                }
                const int zz = nm - k + nr - kr;
                const float g1 = p[1] * (float)(nh + zz), g2 = p[0] * (float)zz;
                const float gpu = g1 + g2;
                float loc = 0.0f;
                if (k)
                {
                    if (lut) { const float tail = k > 8 ? p[3] * (float)(k - 8) : 0.0f; loc = (p[11 + (k < 8 ? k : 8)] + tail) + cx; }
                    else loc = p[2] + c;
                }
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
                const float f = p[4] * (float)(cnt[miss[k - 1]] - 1); const float g = 1.0f + f; const float h = p[3] * g;
                c = c + h;
                const float f2 = p[3] * p[4]; const float h2 = f2 * (float)(cnt[miss[k - 1]] - 1);
                cx = cx + h2;
            }
            const float g1 = p[1] * (float)(nh + nm - k), g2 = p[0] * (float)(nm - k);
            const float gpu = g1 + g2;
            float loc = 0.0f;
            if (k)
            {
                if (lut) { const float tail = k > 8 ? p[3] * (float)(k - 8) : 0.0f; loc = (p[11 + (k < 8 ? k : 8)] + tail) + cx; }
                else loc = p[2] + c;
            }
            const float tt = fmaxf(gpu, loc);
            if (tt < bt - 1e-6f) { bt = tt; best = k; }
        }
    }
    for (int k = 0; k < best; ++k) cpu[miss[k]] = 1;
    const int publish = best + bestr > 0 || p[7] > 0.5f;
    stats[0] += nh; stats[1] += nm + nr; stats[2] += best + bestr; stats[3] += 1;
    int npk = 0;
    if (publish)
        for (int s = 0; s < n; ++s)
        {
            const int64_t e = sel[s] - first;
            if (e < 0 || e >= E || !cpu[e] || !h_nonzero(w[s])) continue;
            const float wf = gflo_h2f(w[s]);
            hpicks[npk * 3] = s / topk;
            hpicks[npk * 3 + 1] = (int32_t)e;
            memcpy(&hpicks[npk * 3 + 2], &wf, 4);
            ++npk;
        }
    for (int s = 0; s < n; ++s)
    {
        const int64_t e = sel[s];
        const int c = e - first >= 0 && e - first < E && cpu[e - first];
        sel_out[s] = (c && !keep_ids) ? -1 : e;
        w_out[s] = c ? 0 : w[s];
    }
    if (publish)
    {
        memcpy(hx, z, sizeof(uint16_t) * (size_t)bsz * H);
        ctrl[2] = li; ctrl[3] = bsz; ctrl[4] = npk;
        ctrl[0] = seq;
        dflag[0] = seq;
    }
    else dflag[0] = 0;
    free(cnt); free(cpu); free(miss); free(rmiss);
}

/* ft_combine_k, trellis build (ft_tier_cu.cu:205-235): a missing done flag is the timeout path (skip the add) */
int gflo_combine(void* out, int is_half, int n, int64_t dflag, const int64_t* ctrl, const float* hout)
{
    if (dflag == 0 || ctrl[1] < dflag) return 0;
    for (int i = 0; i < n; ++i)
    {
        if (is_half)
        {
            uint16_t* o = (uint16_t*)out;
            o[i] = gflo_f2h(gflo_h2f(o[i]) + hout[i]);
        }
        else ((float*)out)[i] += hout[i];
    }
    return 1;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* grouped rows                                                                                                  */
/* ------------------------------------------------------------------------------------------------------------ */

int gflo_grouped_rows(const int64_t* sel, const float* w, int T, int K, const uint8_t* take, int E, int32_t* experts,
                      int32_t* offsets, int32_t* row_token, float* row_weight, int* rows_out)
{
    int32_t* count = (int32_t*)calloc((size_t)E, sizeof(int32_t));
    int32_t* last = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    int32_t* cursor = (int32_t*)calloc((size_t)E, sizeof(int32_t));
    int ret = 0;
    for (int e = 0; e < E; ++e) { last[e] = -1; if (take[e] > 1) ret = -1; }
    for (int t = 0; t < T && ret == 0; ++t)
        for (int k = 0; k < K; ++k)
        {
            const int64_t e = sel[(size_t)t * K + k];
            const float wv = w[(size_t)t * K + k];
            if (!isfinite(wv) || e < -1 || e >= E) { ret = -1; break; }
            if (e == -1) { if (wv != 0.0f) { ret = -1; break; } continue; }
            if (!take[e]) continue;
            if (last[e] == t) { ret = -1; break; }
            last[e] = t;
            ++count[e];
        }
    if (ret == 0)
    {
        int nexp = 0;
        offsets[0] = 0;
        for (int e = 0; e < E; ++e)
            if (count[e])
            {
                experts[nexp] = e;
                cursor[e] = offsets[nexp];
                offsets[nexp + 1] = offsets[nexp] + count[e];
                ++nexp;
            }
        for (int t = 0; t < T; ++t)
            for (int k = 0; k < K; ++k)
            {
                const int64_t e = sel[(size_t)t * K + k];
                if (e < 0 || !take[e]) continue;
                const int32_t row = cursor[e]++;
                row_token[row] = t;
                row_weight[row] = w[(size_t)t * K + k];
            }
        *rows_out = offsets[nexp];
        ret = nexp;
    }
    free(count); free(last); free(cursor);
    return ret;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* router                                                                                                        */
/* ------------------------------------------------------------------------------------------------------------ */

void gflo_route(const float* logits, int M, int E, int topk, int64_t* sel, uint16_t* w)
{
    float* s = (float*)malloc(sizeof(float) * (size_t)E);
    unsigned char* used = (unsigned char*)malloc((size_t)E);
    for (int m = 0; m < M; ++m)
    {
        for (int e = 0; e < E; ++e)
        {
            /* exp evaluated in double and rounded once: the correctly rounded fp32 exp(-x), which the device router
               reproduces exactly (exllamav3's router is not in the reference tree: parity unpinned against it) */
            const float ex = (float)exp(-(double)logits[(size_t)m * E + e]);
            s[e] = 1.0f / (1.0f + ex);
            used[e] = 0;
        }
        float tot = 0.0f;
        float pick[64];
        for (int j = 0; j < topk; ++j)
        {
            int b = -1;
            for (int e = 0; e < E; ++e)
                if (!used[e] && (b < 0 || s[e] > s[b])) b = e;
            used[b] = 1;
            sel[(size_t)m * topk + j] = b;
            pick[j] = s[b];
            tot += s[b];
        }
        for (int j = 0; j < topk; ++j) w[(size_t)m * topk + j] = gflo_f2h(pick[j] / tot);
    }
    free(s); free(used);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* synthetic inputs                                                                                              */
/* ------------------------------------------------------------------------------------------------------------ */

uint64_t gflo_splitmix64_at(uint64_t seed, uint64_t i)
{
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t gflo_seed(int layer, int expert, int proj)
{
    return 0x6A11F1A5ull ^ (((uint64_t)layer << 20) | ((uint64_t)expert << 4) | (uint64_t)proj);
}

void gflo_synth_trellis(uint64_t seed, uint8_t* tr, size_t nbytes)
{
    for (size_t b = 0; b < nbytes; ++b) tr[b] = (uint8_t)(gflo_splitmix64_at(seed, b / 8) >> (8 * (b % 8)));
}

#define SCALE_SALT 0x5C41E50000000000ull

void gflo_synth_scales(uint64_t seed, uint16_t* suh, int k, uint16_t* svh, int n, int fan_in)
{
    const uint64_t s2 = seed ^ SCALE_SALT;
    for (int i = 0; i < k; ++i) suh[i] = (gflo_splitmix64_at(s2, (uint64_t)i) & 1) ? 0xBC00 : 0x3C00;
    const double inv = 1.0 / sqrt((double)fan_in);
    for (int i = 0; i < n; ++i)
    {
        const uint64_t r = gflo_splitmix64_at(s2, (uint64_t)k + (uint64_t)i);
        const double u = (double)(r >> 11) * (1.0 / 9007199254740992.0);
        const double v = ((r & 1) ? -1.0 : 1.0) * (0.5 + u) * inv;
        svh[i] = gflo_f2h((float)v);
    }
}
