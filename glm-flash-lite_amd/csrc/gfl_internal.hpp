// Internal declarations shared by the kernel translation units and the C-ABI host layer.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <utility>
#include <vector>

namespace gfl {

// Kernel timing of profiled stages. While the host layer profiles a stage it points g_kernel_timer (thread-local) at a
// timer; the decode launchers then launch through hipExtLaunchKernelGGL with a start and a stop event that the runtime
// stamps on the kernel's own dispatch, so a stage's time is its kernels' execution without the gaps between packets.
// Each such launch appends one (start, stop) pair. take() hands out a created event, or nullptr.
struct KernelTimer
{
    hipEvent_t (*take)(void* owner);
    void* owner;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pairs;
};
extern thread_local KernelTimer* g_kernel_timer;

template <typename K, typename... A>
inline void timed_launch(K kern, dim3 grid, dim3 block, size_t lds, hipStream_t st, A... args)
{
    if (KernelTimer* t = g_kernel_timer)
    {
        hipEvent_t e0 = t->take(t->owner), e1 = t->take(t->owner);
        if (e0 && e1)
        {
            hipExtLaunchKernelGGL(kern, grid, block, (std::uint32_t)lds, st, e0, e1, 0, args...);
            t->pairs.emplace_back(e0, e1);
            return;
        }
    }
    hipLaunchKernelGGL(kern, grid, block, lds, st, args...);
}

constexpr int MAX_PICKS = 1024;    // tokens * topk per forward call
constexpr int MAX_EXPERTS = 1024;  // experts per layer (ft_split's own limit, ft_tier_cu.cu:260)
constexpr int MAX_TOPK = 16;
constexpr int MAX_GROUPED_PICKS = 65536;  // tokens * topk per prefill (grouped) call
constexpr int LDS_LIMIT = 163840;         // bytes of LDS one workgroup may use on gfx950

// Status words of a context (device int32 array, sticky until gfl_ctx_check reads and clears them).
enum
{
    GFL_STATUS_RELAY_EXPIRED = 0,   // relay turn waits (decode relay launches) that ran out of their bound
    GFL_STATUS_INGRESS_REJECTED = 1,   // published jobs the device worker refused (bad layer, token, expert or weight)
    GFL_STATUS_WORDS = 4,
};
// ints between two last-one counters of the decode launches (act_cnt, out_cnt, blk_cnt): each on a 128-byte line of
// its own. Device-scope atomics on one line are served one after another, and a layer's few hundred arrivals per
// counter line were a measurable part of each launch's tail (config 0: 28.3 against 25.9 us/token).
constexpr int CNT_STRIDE = 32;
constexpr int RELAY_SPIN_DEFAULT = 1 << 22;   // polls of a relay turn wait (s_sleep 1 between polls: ~0.1 s)

// Device-side routing plan of one forward call (all arrays in device memory, capacity cap_slots picks).
struct PlanView
{
    int* hdr;        // [0] union size U, [1] slot count, [2] ids outside [0, E)
    int* uexp;       // [U] expert of union entry u, first-appearance order
    int* uoff;       // [U+1] slot range of union entry u
    int* slot_pick;  // [slots] pick index (token * topk + k) of each slot
    int* slot_u;     // [slots] union entry of each slot
    int* pick_slot;  // [picks] slot of each pick, -1 when skipped
    int* pick_job;   // [picks] reference job index (combine order)
    int* tok_slot;   // [tokens][topk] slots of each token in combine order, -1 padded
    float* tok_w;    // [tokens][topk] their routing weights (fp32)
    int* tok_npk;    // [tokens] number of valid picks of each token
    uint64_t* uptr;  // [U][2] down trellis and svh_down addresses of union entry u (one load for the down launch);
                     // [slots][2], by slot, when the launches run a workgroup per slot (one slot per pass)
    int cap_slots;
};

// gate|up launch: routing plan (published to pv by workgroup 0), gate and/or up GEMV, SwiGLU per 128-block by the
// last workgroup of the block. mat_base/nmat: matrices of this launch (0,2 = both, 0,1 = gate, 1,1 = up). mf = 1:
// MFMA-accumulate GEMV (mode GFL_MODE_MFMA), ns = slots per pass (<= 16); mf = 0: EXACT chain order. rw = 1, 2 or 4
// (EXACT, one slot per pass): the relay launches, a workgroup per (pick, 64 / rw outputs) with rw waves per tile
// column, slot = pick; rw = 0: the per-slot or per-union-entry launches. prio (relay launches only): 1 = each wave
// lowers its issue priority as it progresses, so the waves sharing a SIMD end together; 0 = off; -1 = chosen from the
// launch's waves per SIMD. nsh (relay launches only, else -1 is returned): M shared-expert picks P .. P + M - 1 after
// the routed ones (token p - P, expert row E of ptrs, weight 1), whose down output the combine adds after the token's
// routed sum. gplan (rw = 0 only): the routing plan is
// built once by its own one-workgroup launch before the launch of matrix 0 and read from pv by every workgroup,
// instead of each workgroup building it in LDS.
int launch_gate_up(int K, int ns, const uint64_t* ptrs, int mat_base, int nmat, const int64_t* sel, const void* w,
                   int w_half, int P, int topk, int E, int H, int I, int umax, const uint16_t* x, float* ygu,
                   uint16_t* xtd, int* act_cnt, const float* silu_tab, float act_limit, const PlanView& pv, float* out,
                   int mf, int rw, int prio, int nsh, int gplan, int* status, int spin_max, hipStream_t st);
// down launch: down GEMV + out_block, weighted combine per (token, 128-block) by the token's last expert; mf and ns
// as for launch_gate_up (the same values for both launches of a call). blk_cnt: [cap][H/128] half-block counters of
// the one-slot-per-pass EXACT launch (zero between calls). rw, prio and nsh as for launch_gate_up (rw and nsh the same
// values for both; the relay down launch takes at most 64 routed picks, else -1).
int launch_down(int K, int ns, const uint64_t* ptrs, int topk, int H, int I, int umax, int P, int E, const int64_t* sel,
                const void* w, int w_half, const PlanView& pv, const uint16_t* xtd, float* yd, int* out_cnt,
                int* blk_cnt, float* out, int mf, int rw, int prio, int nsh, int* status, int spin_max,
                hipStream_t st);
size_t gate_up_lds_bytes(int K, int ns, int H, int P, int E, int mf, int rw, int gplan);
size_t down_lds_bytes(int K, int ns, int I, int P, int E, int mf, int rw);
int launch_dequant(const uint8_t* tr, int k, int n, int K, uint16_t* W, hipStream_t st);

// Grouped-rows plan of the prefill path (device arrays; P picks, E experts, M tokens).
struct GPlan
{
    int* hdr;        // [0] slots S, [1] ids outside [-1, E)
    int* cnt;        // [E] slots of each expert
    int* off;        // [E + 1] slot offsets (experts ascending)
    int* slot_pick;  // [P] pick of each slot (picks ascending within an expert)
    int* slot_e;     // [P] expert of each slot
    int* pick_slot;  // [P] slot of each pick, -1 when skipped
    int* pick_c;     // [P] occurrence of the pick among its expert's picks
    int* slot_job;   // [P] reference job number (combine order), set at the slots of job-opening picks
    int* tok_slot;   // [M][topk] slots of each token in combine order
    float* tok_w;    // [M][topk] their routing weights (fp32)
    int* tok_npk;    // [M] valid picks of each token
    int* eord;       // [E] experts in GEMM dispatch order: most slots first, then ascending id
    int* ccnt;       // [chunks][E + 1] picks of each expert per chunk of GP_PLAN_CHUNK picks, other ids at [E]
};

constexpr int GP_PLAN_CHUNK = 1024;   // picks per workgroup of the grouped plan

// Prefill-sized layer forward with MFMA grouped GEMMs (k_prefill.hip): xt [2][cap][H] fp16, ygu [2][cap][I] fp16,
// xd [cap][I] fp16, yraw [cap][H] fp16 workspace, cap >= P. The GEMM outputs ygu and yraw are stored rounded to fp16,
// the first step of the out_block that reads them.
int launch_grouped(const uint64_t* ptrs, const int64_t* sel, const void* w, int w_half, int P, int topk, int E, int H,
                   int I, int Kg, int Ku, int Kd, const uint16_t* x, const GPlan& g, int cap, uint16_t* xt,
                   uint16_t* ygu, uint16_t* xd, uint16_t* yraw, const float* silu_tab, float act_limit, float* out,
                   hipStream_t st);
size_t grouped_gemm_lds_bytes(int K);
// EXACT layer forward at prefill sizes (k_prefill.hip), bit-identical to the decode path: the grouped plan, the
// input transforms as fp32 in the accumulator-chain layout, the reference's accumulator chains with each weight
// decoded once per pass of up to 64 of an expert's slots, SwiGLU, the combine in job order. xt [2][cap][H] fp32,
// ygu [2][cap][I] fp16, xd [cap][I] fp32, yraw [cap][H] fp16 workspace, cap >= P, cap * max(H, I) * 4 < 2^31
// (else -1, nothing launched).
int launch_exact_chains(const uint64_t* ptrs, const int64_t* sel, const void* w, int w_half, int P, int topk, int E,
                        int H, int I, int Kg, int Ku, int Kd, const uint16_t* x, const GPlan& g, int cap, float* xt,
                        uint16_t* ygu, float* xd, uint16_t* yraw, const float* silu_tab, float act_limit, float* out,
                        hipStream_t st);
// The grouped plan alone (first three launches of launch_grouped): slots, offsets, job order per token.
void launch_grouped_plan(const int64_t* sel, const void* w, int w_half, int P, int topk, int E, const GPlan& g,
                         hipStream_t st);

int launch_split(const int64_t* sel, const uint16_t* w, const uint16_t* z, int n, int bsz, int topk, int H, int E,
                 int first, const int32_t* slotof, const float* score, const float* pol, int64_t* ctrl, uint16_t* hx,
                 int32_t* hpicks, int64_t seq, int li, int keep_ids, int64_t* sel_out, uint16_t* w_out,
                 int64_t* dflag, int64_t* stats, const int32_t* rres, hipStream_t st);
void launch_combine(void* out, int is_half, int n, const int64_t* dflag, const int64_t* ctrl, const float* hout,
                    int64_t* stats, int64_t timeout_ns, hipStream_t st);
void launch_synth(uint8_t* dst, size_t nbytes, uint64_t seed, hipStream_t st);
// device worker (k_split.hip): the published job as a selection sel [bsz][topk] / w fp32 (state = {accepted, seq}),
// and the done word once the forward on it has written hout
void launch_ingress_take(const int64_t* ctrl, const int32_t* hpicks, int li, int bsz, int topk, int E, int64_t* sel,
                         float* w, int64_t* state, int* status, hipStream_t st);
void launch_ingress_answer(int64_t* ctrl, const int64_t* state, hipStream_t st);
int launch_route(const float* logits, int M, int E, int topk, int64_t* sel, uint16_t* w, hipStream_t st);
int launch_route_split(const float* logits, int M, int ER, int topk, int64_t* sel, uint16_t* w, const uint16_t* z,
                       int H, int E, int first, const int32_t* slotof, const float* score, const float* pol,
                       int64_t* ctrl, uint16_t* hx, int32_t* hpicks, int64_t seq, int li, int keep_ids,
                       int64_t* sel_out, uint16_t* w_out, int64_t* dflag, int64_t* stats, const int32_t* rres,
                       hipStream_t st);

}  // namespace gfl
