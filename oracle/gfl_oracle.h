/* CPU oracle for the routed-MoE expert path (test infrastructure only).
 *
 * This is the checker the HIP path is compared against. It restates, in plain C, the reference's EXL3 trellis
 * decode, its Hadamard/activation rounding points, its EXACT/AFFINE expert GEMVs, the MoE job build and combine,
 * the ft_split/ft_combine semantics and the grouped-rows builder. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may call it; the product library never links it.
 *
 * Reference citations are paths relative to the reference repository root.
 */
#ifndef GFL_ORACLE_H
#define GFL_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 helpers (software round-to-nearest-even; F16C-free) ---- */
float gflo_h2f(uint16_t h);
uint16_t gflo_f2h(float f);
float gflo_r16(float f);

/* ---- format (kernels/cpu_avx2/ft_core.h:28-83) ---- */
/* 16-bit trellis state of stream index t (0..255) of one tile of K bits/weight (tile = 16*K uint16 = 32*K bytes).
 * K-generic form of state_scalar (ft_core.h:65-73); identical to it at K=3. */
uint16_t gflo_state(const uint16_t* packed, int K, int t);
/* stream index -> r*16 + c inside the 16x16 tile (init_perm, ft_core.h:50-61) */
int gflo_perm(int i);
/* byte sum of st*MUL1 mod 2^32 (bytesum, ft_core.h:75-79) */
int gflo_bytesum(uint16_t st);
/* codebook weight as fp16 bits: round16(fma(1024+bytesum, KINV, KBIAS)) (w_gpu, ft_core.h:82) */
uint16_t gflo_weight_bits(uint16_t st);
/* Full dequant of one matrix (tiles row-major [k/16][n/16], 32*K bytes each) to fp16 bits W[k][n]
 * (dense_weights, ft_core.h:1657-1672). */
void gflo_dequant(const uint8_t* tr, int k, int n, int K, uint16_t* W);

/* ---- transforms (ft_core.h:89-132) ---- */
void gflo_had128(float* v);
void gflo_prep_block(const float* x, const uint16_t* suh, float* xt);
void gflo_out_block(float* y, const uint16_t* svh);
float gflo_act_mul(float g, float u, float limit);

/* ---- GEMV of one matrix for M tokens ---- */
/* xt: [M][k] transformed activations (fp16-valued fp32); y: [M][n] raw (pre out_block) fp32.
 * mode 1 = EXACT (tile_accum<EXACT> lane order and FMA chain, ft_core.h:313-387),
 * mode 0 = AFFINE (KINV*sum(s*x) + CAFF*sum(x), ft_core.h:383). */
void gflo_gemv(const uint8_t* tr, int k, int n, int K, const float* xt, int M, float* y, int mode,
               const float* sumx);
/* sumx (AFFINE only): per-token sum of xt, or NULL for a running sum in element order (the gate/up association,
 * ft_core.h:947); the down projection passes per-128-block partial sums added in block order (ft_core.h:987,1003). */

/* one matrix = trellis + input/output sign/scale vectors */
typedef struct { const uint8_t* tr; const uint16_t* suh; const uint16_t* svh; int k, n, K; } gflo_mat;
typedef struct { gflo_mat g, u, d; } gflo_expert;

/* One expert on M tokens of x [M][H] (fp16-valued fp32): prep -> gate/up -> out_block -> act -> prep -> down ->
 * out_block (fwd_phase phases 0-2, ft_core.h:933-1019). y: [M][H]. */
void gflo_expert_forward(const gflo_expert* E, const float* x, int M, float* y, int mode, float act_limit);
/* fp64-accumulated reference expert (ref_linear/ref_expert, ft_core.h:1674-1691), one token */
void gflo_expert_ref64(const gflo_expert* E, const float* x, float* y, float act_limit);

/* ---- MoE layer forward (moe_forward, ft_core.h:1338-1407) ----
 * route: per token t, topk entries (sel[t*topk+j] < 0 skipped) with fp32 weights.
 * Jobs in first-appearance order, <= 8 tokens per job; out[t] = sum over jobs in order of w * expert(x_t). */
int gflo_moe_forward(const gflo_expert* experts, int E, const float* x, int ntok, const int32_t* sel,
                     const float* w, int topk, float* out, int mode, float act_limit);
/* The same with the jobs built over all ntok tokens (so every token's combine order is the full batch's) but only
 * the rows with want[t] != 0 evaluated; the other rows of out are zero. want = NULL: all rows. */
int gflo_moe_forward_rows(const gflo_expert* experts, int E, const float* x, int ntok, const int32_t* sel,
                          const float* w, int topk, const uint8_t* want, float* out, int mode, float act_limit);
/* job list as the reference builds it: returns job count; job_e[j], job_m[j], job_tok[j*8+i], job_w[j*8+i] */
int gflo_build_jobs(int E, int ntok, const int32_t* sel, const float* w, int topk, int32_t* job_e, int32_t* job_m,
                    int32_t* job_tok, float* job_w);

/* ---- split / combine (kernels/cpu_avx2/ft_tier_cu.cu:21-236, kernels/k110/ft_split_fast.cu:18-198) ----
 * ctrl: host-visible int64[>=5]; hx: fp16 [bsz*H]; hpicks: int32 [n*3]. rres may be NULL. All outputs in place. */
void gflo_split(const int64_t* sel, const uint16_t* w, const uint16_t* z, int n, int bsz, int topk, int H, int E,
                int first, const int32_t* slotof, const float* score, const float* p, int64_t* ctrl, uint16_t* hx,
                int32_t* hpicks, int64_t seq, int li, int keep_ids, int64_t* sel_out, uint16_t* w_out,
                int64_t* dflag, int64_t* stats, const int32_t* rres);
/* out += hout when dflag != 0 and the done flag ctrl[1] >= dflag (is_half: out holds fp16 bits).
 * returns 1 if added, 0 if skipped. */
int gflo_combine(void* out, int is_half, int n, int64_t dflag, const int64_t* ctrl, const float* hout);

/* ---- grouped rows (kernels/cpu_avx2/ft_tier_ext.cpp:1047-1097) ----
 * sel int64 [T*K], w fp32 [T*K], take uint8 [E] -> experts [nexp], offsets [nexp+1], row_token, row_weight.
 * returns nexp, or -1 on a rejected input (duplicate expert for a token, index out of range, masked pick with w!=0,
 * nonfinite weight, take entry > 1). *rows_out receives the row count. */
int gflo_grouped_rows(const int64_t* sel, const float* w, int T, int K, const uint8_t* take, int E, int32_t* experts,
                      int32_t* offsets, int32_t* row_token, float* row_weight, int* rows_out);

/* ---- router (exllamav3 sigmoid top-k, renormalised, fp16 weights) ----
 * logits fp32 [M][E] -> sel int64 [M][topk], w fp16 bits [M][topk]; ties resolved to the lower expert index. */
void gflo_route(const float* logits, int M, int E, int topk, int64_t* sel, uint16_t* w);

/* ---- synthetic inputs (splitmix64, counter form) ---- */
uint64_t gflo_splitmix64_at(uint64_t seed, uint64_t i);
uint64_t gflo_seed(int layer, int expert, int proj);
void gflo_synth_trellis(uint64_t seed, uint8_t* tr, size_t nbytes);
/* suh: Rademacher +-1; svh: +-U(0.5,1.5)/sqrt(fan_in) rounded to fp16 */
void gflo_synth_scales(uint64_t seed, uint16_t* suh, int k, uint16_t* svh, int n, int fan_in);

#ifdef __cplusplus
}
#endif
#endif
