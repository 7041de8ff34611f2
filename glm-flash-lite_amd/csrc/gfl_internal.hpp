// Internal declarations shared by the kernel translation units and the C-ABI host layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gfl {

constexpr int MAX_PICKS = 1024;    // tokens * topk per forward call
constexpr int MAX_EXPERTS = 1024;  // experts per layer (ft_split's own limit, ft_tier_cu.cu:260)
constexpr int MAX_TOPK = 16;

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
    int cap_slots;
};

void launch_plan(const int64_t* sel, const void* w, int w_half, int P, int topk, int E, const PlanView& pv,
                 hipStream_t st);
int launch_chain(int K, int ns, bool prep, const uint64_t* ptrs, int mat_base, int nmat, int kdim, int ndim,
                 const PlanView& pv, int topk, int umax, const uint16_t* xin, float* yout, hipStream_t st);
void launch_act(const uint64_t* ptrs, const PlanView& pv, int smax, const float* ygu, uint16_t* xtd, int I,
                float limit, const float* exp_tab, hipStream_t st);
void launch_final(const uint64_t* ptrs, const PlanView& pv, const void* w, int w_half, int M, int topk,
                  const float* yd, float* out, int H, hipStream_t st);
int launch_dequant(const uint8_t* tr, int k, int n, int K, uint16_t* W, hipStream_t st);

int launch_split(const int64_t* sel, const uint16_t* w, const uint16_t* z, int n, int bsz, int topk, int H, int E,
                 int first, const int32_t* slotof, const float* score, const float* pol, int64_t* ctrl, uint16_t* hx,
                 int32_t* hpicks, int64_t seq, int li, int keep_ids, int64_t* sel_out, uint16_t* w_out,
                 int64_t* dflag, int64_t* stats, const int32_t* rres, hipStream_t st);
void launch_combine(void* out, int is_half, int n, const int64_t* dflag, const int64_t* ctrl, const float* hout,
                    int64_t* stats, int64_t timeout_ns, hipStream_t st);
void launch_synth(uint8_t* dst, size_t nbytes, uint64_t seed, hipStream_t st);

}  // namespace gfl
