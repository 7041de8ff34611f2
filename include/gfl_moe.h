/* gfl_moe -- MI355X (gfx950) routed-MoE expert path behind a C ABI.
 *
 * Drop-in for the routed-expert path of glm-flash-lite: the ft_split / ft_combine kernels the k_ftsplit and cpu_tier
 * monkeypatches call, the expert-call signature of the CPU tier (tier_init / tier_add_layer / tier_forward) and the
 * expert-residency lookup of expert_cache. With every expert resident in HBM the host tier and the PCIe cache are
 * gone; what remains is the EXL3 trellis decode + Hadamard SwiGLU expert arithmetic and the split/combine around it.
 *
 * Conventions: plain pointers and sizes, no framework types. Device pointers unless stated otherwise. Every call that
 * launches work takes a stream (a hipStream_t; NULL = the null stream), is stream-ordered and never synchronises the
 * host. Return value 0 = success; otherwise a GFL_E* code with a message in gfl_last_error() (thread-local).
 * Citations are paths in the reference repository.
 */
#ifndef GFL_MOE_H
#define GFL_MOE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gfl_ctx gfl_ctx;
typedef void* gfl_stream; /* hipStream_t */

enum
{
    GFL_OK = 0,
    GFL_EINVAL = 1,   /* bad argument (shape, dtype code, unregistered layer, unsupported K) */
    GFL_ERUNTIME = 2, /* HIP runtime error */
    GFL_ENOMEM = 3,   /* device allocation failed */
    GFL_EUNSUPPORTED = 4, /* gfl_moe_forward_shared: this call cannot run the shared expert in the routed launches;
                           * nothing was launched (the caller runs the two calls itself) */
};

/* Expert arithmetic modes, numbered as tier_forward's `mode` (kernels/cpu_avx2/ft_tier_ext.cpp:865-904).
 * The device path computes EXACT (bit-identical to the reference's EXACT mode) for AUTO, EXACT, AFFINE and I16: the
 * last two name the reference CPU engine's speed modes, and EXACT lies closer to the fp64 expert than either.
 * GFL_MODE_MFMA has no counterpart in the reference: the same bit-exact weights, transforms, rounding points and
 * combine order, with the GEMV sums over the hidden dimension formed by MFMAs (fp32 accumulate) instead of EXACT's
 * chains, for callers that trade bit-exactness for speed. Its outputs differ from EXACT by accumulation rounding
 * carried through the fp16 rounding points (max-abs about 1e-3..3e-3 of the output RMS, as far as the reference's own
 * fp64 expert lies from EXACT), so it is outside the 2e-3 bar that EXACT meets by construction. */
enum
{
    GFL_MODE_AUTO = -1,
    GFL_MODE_AFFINE = 0,
    GFL_MODE_EXACT = 1,
    GFL_MODE_I16 = 2,
    GFL_MODE_MFMA = 3,
};

/* Last error message of the calling thread ("" if none). */
const char* gfl_last_error(void);
/* ABI version (major*100 + minor). */
int gfl_version(void);

/* Context on one device: registered layers plus the per-call workspace.
 * Replaces the global Tier singleton of tier_init (kernels/cpu_avx2/ft_tier_ext.cpp:137-157).
 * One stream per context: calls that overlap on two streams share the context's plan, workspace and counters and
 * race. Workspaces are never freed before gfl_ctx_destroy, so a HIP graph captured from any call stays valid. */
int gfl_ctx_create(int device, gfl_ctx** out);
int gfl_ctx_destroy(gfl_ctx* ctx);

/* Whether other GPU work runs beside this context's decode calls (shared != 0), such as a shared expert on a side
 * stream. No counterpart in the reference: it selects launch shapes only, never results (every shape is bit-exact).
 * With shared = 0 (the default) a call of 769..1536 gate|up tile columns (8 picks at I = 1536) runs the relay
 * launches, which put 3 waves on every SIMD, and a call of up to 768 (e.g. one expert) 4 waves per tile column; with
 * shared != 0 the first keeps the per-slot launches and the second takes 2 waves per gate|up column and 1 per down
 * column, which leave SIMDs free for the other work. Read at each gfl_moe_forward / gfl_moe_forward_noalloc call (and so fixed in a captured
 * graph). */
int gfl_ctx_set_shared(gfl_ctx* ctx, int shared);

/* Synchronises the context's device, then reads and clears its status words, which count since the last check:
 * relay hand-off waits of the decode launches that ran out of their bound (the outputs of the calls concerned are
 * wrong), and published jobs that gfl_ingress_serve refused. Returns GFL_ERUNTIME with the counts in
 * gfl_last_error() when either is nonzero, else GFL_OK. The reference's counterpart of a worker failure is an
 * exception out of tier_forward or the LUT worker's failed word ctrl[7] (kernels/cpu_avx2/ft_tier_ext.cpp:744-775);
 * these conditions arise on the device, so they are collected there and surfaced here. The relay wait's bound is
 * 2^22 polls (about 0.1 s); the environment variable GFL_RELAY_SPIN_LIMIT, read by gfl_ctx_create, lowers it (0 makes
 * every wait expire: only for testing this report). */
int gfl_ctx_check(gfl_ctx* ctx);

/* Largest hidden or intermediate size a layer may have: every trellis matrix then stays below 2^31 bytes (at most
 * 32768 x 32768 x 5/8), so the kernels' 32-bit buffer offsets cannot wrap. */
#define GFL_MAX_DIM 32768

/* Register layer `li`: E experts of a SwiGLU MLP, hidden H, intermediate I (multiples of 256 up to GFL_MAX_DIM);
 * gate/up are [H->I], down [I->H], each an EXL3 trellis of K bits per weight (k_gate/k_up/k_down in 2..5) in 16x16
 * tiles stored row-major [k/16][n/16].
 * ptrs: HOST array [E][9] of DEVICE addresses per expert:
 *   trellis gate, up, down; suh_gate, svh_gate, suh_up, svh_up, suh_down, svh_down (fp16 sign/scale vectors).
 * Trellis addresses must be 4-byte aligned, suh/svh addresses 16-byte aligned (both hold for torch allocations).
 * The table is copied; the weights stay where the caller put them (full HBM residency).
 * Replaces tier_add_layer (ft_tier_ext.cpp:160-211) and the pointer tables expert_cache maintains
 * (glm53/expert_cache.py:540-635). */
int gfl_register_layer(gfl_ctx* ctx, int li, int E, int H, int I, int k_gate, int k_up, int k_down,
                       const uint64_t* ptrs);
/* (Registration also reserves the decode workspace for 1024 picks at the largest registered H and I, so that
 * gfl_moe_forward never allocates.) */

/* Shape of a registered layer: info[6] = {E, H, I, k_gate, k_up, k_down} (host array). The forward calls take no
 * shape arguments, so callers check their x / out widths against H with it (tier_forward checks x.size(1) == H,
 * ft_tier_ext.cpp:865-904). No counterpart of its own in the reference. */
int gfl_layer_info(gfl_ctx* ctx, int li, int* info);

/* Routed-expert forward of one layer (the expert call, tier_forward, ft_tier_ext.cpp:865-904):
 *   out[t] = sum over picks k of w[t,k] * expert_{sel[t,k]}(x[t]), picks with sel < 0 skipped,
 * summed in the reference's job order (moe_forward, kernels/cpu_avx2/ft_core.h:1338-1407).
 * x: fp16 [M, H]; sel: int64 [M, topk]; w: [M, topk] fp16 (w_is_half=1) or fp32; out: fp32 [M, H].
 * act_limit: SwiGLU clamp (tier_set_act_limit, ft_tier_ext.cpp:629-636), 0 = off. topk <= 16; x 16-byte aligned.
 * Empty calls, as the reference's tier_forward takes them (ft_tier_ext.cpp:893-903): M = 0 does nothing (every
 * buffer may be NULL); topk = 0 writes M rows of zeros to out (sel and w may be NULL).
 * M*topk <= 1024: the decode launches (routing plan built in every workgroup). 1024 < M*topk <= 65536 (EXACT modes
 * only; MFMA is refused there): the grouped plan of the prefill path, then the reference's accumulator chains (each
 * chain step one element of a K=1 fp32 MFMA, i.e. an fmaf), each weight decoded once per pass of up to 64 of an
 * expert's slots, bit-identical to the reference's EXACT mode at any batch size; there out must be 16-byte aligned
 * too and M*topk*max(H, I) < 2^29. That path uses the prefill workspace (gfl_grouped_reserve sizes it ahead of graph
 * capture; otherwise the first call of a larger size grows it). */
int gfl_moe_forward(gfl_ctx* ctx, int li, const uint16_t* x, const int64_t* sel, const void* w, int w_is_half, int M,
                    int topk, float* out, int mode, float act_limit, gfl_stream stream);

/* The shared expert of layer li, for gfl_moe_forward_shared: ptr_row = its 9 device addresses, as one row of
 * gfl_register_layer's table; k_*: its bit widths. Replaces an earlier one; gfl_register_layer for li drops it. The
 * reference runs the shared GatedMLP beside the routed experts on a side stream (glm53/k_overlap.py:61-90); this has
 * no counterpart of its own there. Like gfl_register_layer, not to be called while a graph that runs li is captured
 * or replayed (the layer's table moves). */
int gfl_register_shared(gfl_ctx* ctx, int li, int k_gate, int k_up, int k_down, const uint64_t* ptr_row);

/* out[t] = routed layer li (as gfl_moe_forward) + its shared expert for x[t] (weight 1), added in fp32 after the
 * routed sum: bit-identical to gfl_moe_forward into out followed by out += shared(x), the join of glm53/k_overlap.py.
 * act_limit clamps the shared expert's SwiGLU as it does the routed experts'.
 * The shared expert rides on the routed call's two launches as one more pick per token, so the pair costs about one
 * routed call of M*(topk+1) picks. That needs the relay launches (EXACT modes, M*topk <= 64, topk >= 1, a context
 * not set shared at 769..1536 gate|up columns) and the shared expert's bit widths equal to the layer's; any other
 * call returns GFL_EUNSUPPORTED with nothing launched. GFL_EINVAL if the layer has no shared expert. */
int gfl_moe_forward_shared(gfl_ctx* ctx, int li, const uint16_t* x, const int64_t* sel, const void* w, int w_is_half,
                           int M, int topk, float* out, int mode, float act_limit, gfl_stream stream);

/* No counterpart in the reference. gfl_moe_forward with the per-call workspace in a file-scope device array of the
 * library (about 7.8 MiB per device, held until the process ends) instead of the context's reserved workspace: for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). It calls no hipMalloc, hipFree or other allocating routine (and records no profiling events);
 * everything it needs was allocated by gfl_ctx_create and gfl_register_layer. Same arguments and results as
 * gfl_moe_forward (bit-identical), within the array's layout: M*topk <= GFL_NOALLOC_MAX_PICKS, the layer's
 * H <= GFL_NOALLOC_MAX_H and I <= GFL_NOALLOC_MAX_I, else GFL_EINVAL. All calls on one device share the array (its
 * counters are cleared on the device's first call and left at zero by every call). Eager calls from any context or
 * stream on one device are ordered through a per-device event (each waits for the previous call and records its own
 * end), so they run one after another. A call captured into a HIP graph is ordered only inside that graph: replays
 * of it that overlap other calls on the device, eager or replayed, race. */
#define GFL_NOALLOC_MAX_PICKS 64
#define GFL_NOALLOC_MAX_H 8192
#define GFL_NOALLOC_MAX_I 4096
int gfl_moe_forward_noalloc(gfl_ctx* ctx, int li, const uint16_t* x, const int64_t* sel, const void* w,
                            int w_is_half, int M, int topk, float* out, int mode, float act_limit, gfl_stream stream);

/* mode: AUTO, AFFINE, EXACT or I16 (all computed bit-exact to EXACT), or MFMA. With MFMA the workgroups of a routed expert take up to 4 of its slots
 * per pass, so the expert's tiles are decoded once for all of them.
 * Environment: GFL_SLOTS_PER_PASS = 1, 2, 4 or 8 forces the number of (token, expert) slots one GEMV pass of
 * gfl_moe_forward accumulates (default: 1 up to M = 8, with a workgroup per slot; else 2, with a workgroup per expert
 * whose slots take passes; MFMA: min(M, 4)). Read once by gfl_ctx_create. */

/* Routed-expert forward of one layer for prefill-sized M (the north star's MFMA grouped GEMM), same arguments and
 * result layout as gfl_moe_forward: x fp16 [M, H], sel int64 [M, topk] (ids outside [0, E) skipped), w fp16 or fp32
 * [M, topk], out fp32 [M, H]; M*topk <= 65536 and M*topk*max(H, I) < 2^30; x and out 16-byte aligned; M = 0 and
 * topk = 0 as in gfl_moe_forward. Rows are
 * grouped expert-major (tier_lut_build_grouped_rows, kernels/cpu_avx2/ft_tier_ext.cpp:1047-1097), gate|up and down
 * run as v_mfma_f32_16x16x32_f16 grouped GEMMs on the bit-exact dequantized fp16 weights, the transforms keep the
 * reference's fp16 rounding points and the combine its job order (kernels/cpu_avx2/ft_core.h:933-1033). The
 * hidden-dimension sums are formed in MFMA order, so results differ from the EXACT mode of gfl_moe_forward by fp32
 * accumulation rounding (max-abs up to about 3.6e-3 of the output RMS, as far as the reference's own fp64 expert,
 * ref_expert, ft_core.h:1674-1691, lies from EXACT): outside the 2e-3 bar, so this is an explicit opt-in that no
 * reference mode number reaches (tier_forward and gfl_moe_forward compute EXACT at every size). Profiling stage 2. */
int gfl_grouped_forward(gfl_ctx* ctx, int li, const uint16_t* x, const int64_t* sel, const void* w, int w_is_half,
                        int M, int topk, float* out, float act_limit, gfl_stream stream);

/* Size the prefill workspace (gfl_grouped_forward, gfl_grouped_plan and gfl_moe_forward above 1024 picks) for calls
 * of up to max_picks picks on every layer registered so far, so that later calls (and HIP graph captures of them)
 * allocate nothing. Without it the first call of a larger size grows the workspace (never during a capture). No
 * counterpart in the reference. */
int gfl_grouped_reserve(gfl_ctx* ctx, int max_picks);

/* The routing plan of gfl_grouped_forward alone, copied out of the context's workspace (all device pointers; no
 * counterpart in the reference: it exposes the device's grouped rows and combine order so that they can be checked
 * against tier_lut_build_grouped_rows, ft_tier_ext.cpp:1047-1097, and moe_forward's job order,
 * kernels/cpu_avx2/ft_core.h:1343-1349). sel int64 [M*topk], w fp16 (w_is_half) or fp32 [M*topk], E <= 1024.
 * hdr int32 [2] = {slots S, ids outside [-1, E)}; off int32 [E+1] slot offsets (experts ascending); slot_pick and
 * slot_e int32 [M*topk] (first S valid) = each slot's pick and expert, picks ascending within an expert; tok_slot
 * int32 and tok_w fp32 [M][topk] = each token's slots and weights in (job, pick) order, first tok_npk[t] valid;
 * tok_npk int32 [M]. */
int gfl_grouped_plan(gfl_ctx* ctx, const int64_t* sel, const void* w, int w_is_half, int M, int topk, int E,
                     int* hdr, int* off, int* slot_pick, int* slot_e, int* tok_slot, float* tok_w, int* tok_npk,
                     gfl_stream stream);

/* Dequantize one trellis matrix to fp16 W[k][n] (dense_weights, kernels/cpu_avx2/ft_core.h:1657-1672). */
int gfl_dequant(const void* trellis, int k, int n, int K, uint16_t* out, gfl_stream stream);

/* ft_split (kernels/cpu_avx2/ft_tier_cu.cu:238-271, kernels/k110/ft_split_fast.cu:200-235), same arguments with
 * tensors as pointers: sel int64 [n], w fp16 [n], z fp16 [bsz, H], slotof int32 [E], score fp32 [E], pol fp32 [20],
 * ctrl int64 [>=5] / hx fp16 [bsz*H] / hpicks int32 [n*3] (host-mapped or device memory), sel_out int64 [n],
 * w_out fp16 [n], dflag int64 [1], stats int64 [8], rres int32 [E] or NULL. n = bsz*topk <= 1024, E <= 1024.
 * Outputs are the reference's bit for bit, including its handshake: a published job (ctrl[0] = seq, dflag = seq) is
 * answered by its consumer, a reference host worker (worker_main, ft_tier_ext.cpp:781-802) or the device worker
 * gfl_ingress_serve, never by the split itself. Scores must be finite (the reference's two split kernels order NaN
 * scores differently from each other). */
int gfl_split(const int64_t* sel, const uint16_t* w, const uint16_t* z, int bsz, int n, int H, int E, int first,
              const int32_t* slotof, const float* score, const float* pol, int64_t* ctrl, uint16_t* hx,
              int32_t* hpicks, int64_t seq, int li, int keep_ids, int64_t* sel_out, uint16_t* w_out, int64_t* dflag,
              int64_t* stats, const int32_t* rres, gfl_stream stream);

/* Router and split: the routing_fn that cpu_tier.routed wraps (glm53/cpu_tier.py:305-333) followed by ft_split on
 * its output. logits fp32 [M, E_route] -> sel int64 [M, topk] / w fp16 [M, topk] (written: the routing gfl_route
 * computes), then the split of those picks with the remaining arguments as gfl_split's (bsz = M,
 * n = M * topk <= 1024). One launch up to M = 4 (a wave per token); above, gfl_route's launch then gfl_split's, with
 * the same results. No counterpart of its own in the reference (it fuses two of its launches). */
int gfl_route_split(const float* logits, int M, int E_route, int topk, int64_t* sel, uint16_t* w, const uint16_t* z,
                    int H, int E, int first, const int32_t* slotof, const float* score, const float* pol,
                    int64_t* ctrl, uint16_t* hx, int32_t* hpicks, int64_t seq, int li, int keep_ids, int64_t* sel_out,
                    uint16_t* w_out, int64_t* dflag, int64_t* stats, const int32_t* rres, gfl_stream stream);

/* ft_combine (kernels/cpu_avx2/ft_tier_cu.cu:273-294): when dflag != 0 wait (at most timeout_ns) for the done word
 * ctrl[1] >= dflag, then out += hout. out fp32 or fp16 (out_is_half) [n]; stats as ft_split's (4 wait ns, 5 waits,
 * 6 timeouts, 7 already done). */
int gfl_combine(void* out, int out_is_half, int n, const int64_t* dflag, const int64_t* ctrl, const float* hout,
                int64_t* stats, int64_t timeout_ns, gfl_stream stream);

/* The device worker: run_job + worker_main's answer (kernels/cpu_avx2/ft_tier_ext.cpp:400-627, 781-802) on the
 * device, stream-ordered after the split that published the job. When a job is pending (ctrl[0] != ctrl[1]):
 * hout[t] = sum over its ctrl[4] picks (token, expert, fp32 weight bits, in hpicks) of w * expert(hx[t]) for layer li,
 * in the reference's job order, rows of tokens without picks zeroed (run_job zeroes hout for an empty job), then the
 * done word ctrl[1] = ctrl[0] (system-scope release after hout). Every expert is resident, so every job is computed.
 * The job must name layer li (ctrl[2]), ntok = ctrl[3] <= bsz tokens and at most topk picks per token, with tokens and
 * experts in range; a job that does not is left unanswered (gfl_combine then times out and counts it) and counted in
 * the status words (gfl_ctx_check). No pending job: hout's bsz rows are zeroed and nothing is answered.
 * hx fp16 [bsz, H] (16-byte aligned), hpicks int32 [bsz*topk][3], hout fp32 [bsz, H], ctrl int64 [>= 5]: the
 * buffers gfl_split published to (host-mapped or device memory). bsz*topk <= 1024; mode -1..2 (computed EXACT, as
 * gfl_moe_forward). Only one consumer may serve a ctrl block: do not run a host worker on the same ctrl. */
int gfl_ingress_serve(gfl_ctx* ctx, int li, int bsz, int topk, int64_t* ctrl, const uint16_t* hx,
                      const int32_t* hpicks, float* hout, int mode, float act_limit, gfl_stream stream);

/* Expert-major routing rows (tier_lut_build_grouped_rows, ft_tier_ext.cpp:1047-1097), HOST arrays:
 * sel int64 [T*K], w fp32 [T*K], take uint8 [E] -> experts [<=E], offsets [<=E+1], row_token / row_weight [<=T*K].
 * Returns the expert count (>= 0) or -GFL_EINVAL on a rejected routing; *rows receives the row count. */
int gfl_grouped_rows(const int64_t* sel, const float* w, int T, int K, const uint8_t* take, int E, int32_t* experts,
                     int32_t* offsets, int32_t* row_token, float* row_weight, int* rows);

/* Router for the split (the model's routing_fn that cpu_tier.routed calls first, glm53/cpu_tier.py:305-307; exllamav3's
 * own router is not in the reference tree): logits fp32 [M, E] (finite) -> sel int64 [M, topk], w fp16 [M, topk], all
 * device memory. Scores s = 1 / (1 + e) in fp32 with e = exp(-x) correctly rounded to fp32; the topk largest scores in
 * order (lower expert index on ties); w = s / (sum of the picked scores, added in pick order) rounded to fp16.
 * E <= 1024, topk <= min(E, 64). One wave per token, stream-ordered. */
int gfl_route(const float* logits, int M, int E, int topk, int64_t* sel, uint16_t* w, gfl_stream stream);

/* Fill nbytes of device memory with the splitmix64 stream of `seed` (synthetic trellis for tests and benchmarks;
 * any bit stream is a valid EXL3 tile). Byte b = byte (b % 8) of output b/8. */
int gfl_synth_trellis(void* dst, size_t nbytes, uint64_t seed, gfl_stream stream);

/* The SwiGLU gate exponential, host copy: out[b] = expf(-g) for every fp16 bit pattern b of g (n >= 65536 floats).
 * silu (kernels/cpu_avx2/ft_core.h:123) calls the host C library's expf; g is always fp16-valued, so the gate is
 * tabulated from this table, evaluated with that same library call. */
int gfl_exp_table(float* out, int n);

/* The SwiGLU gate, host copy: out[b] = g / (1.0f + expf(-g)) in fp32 (one rounded add, one rounded division, as
 * ft_core.h:123 evaluates it) for every fp16 bit pattern b of g (n >= 65536 floats). Every context uploads this table
 * and the activation kernels read it. No counterpart in the reference: it exposes the table for checking. */
int gfl_silu_table(float* out, int n);

/* Host-side counters of the context (no device sync): [0] forward calls, [1] picks submitted, [2] registered layers,
 * [3] workspace bytes. Writes min(n, 4) entries into the host array `out`. */
int gfl_stats(gfl_ctx* ctx, int64_t* out, int n);

/* Per-stage device timing of gfl_moe_forward, the counterpart of the per-phase wall times tier_stats reports
 * (ft_tier_ext.cpp:906-914): while enabled, every forward brackets its launches with device events. Stage 1 is the
 * gate|up launch (routing plan, gate|up GEMV, SwiGLU and down-input prep), stage 3 the down launch (down GEMV,
 * output transform, weighted combine); stage 2 is a whole gfl_grouped_forward call (its eight launches); stages 0 and
 * 4 (plan, combine) run inside the other launches and stay 0.
 * gfl_profile_read synchronises the recorded events, adds their elapsed milliseconds into stage_ms[5] and launch
 * counts into launches[5] (host arrays), and clears the record. */
int gfl_profile_enable(gfl_ctx* ctx, int enable);
int gfl_profile_read(gfl_ctx* ctx, double* stage_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif
#endif
