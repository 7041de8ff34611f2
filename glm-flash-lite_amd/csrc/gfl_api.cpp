// C-ABI host layer of gfl_moe (include/gfl_moe.h): argument checks, layer registry, workspace, kernel dispatch.
#include "gfl_moe.h"
#include "gfl_internal.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

namespace gfl {
thread_local KernelTimer* g_kernel_timer = nullptr;
}

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg)
{
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what)
{
    return fail(GFL_ERUNTIME, std::string(what) + ": " + hipGetErrorString(e));
}

#define GFL_HIP(call)                                       \
    do                                                      \
    {                                                       \
        hipError_t e_ = (call);                             \
        if (e_ != hipSuccess) return hip_fail(e_, #call);   \
    } while (0)

struct Layer
{
    int E = 0, H = 0, I = 0, K[3] = { 0, 0, 0 };
    uint64_t* dptrs = nullptr;  // device copy of the [E][9] table, [E + 1][9] with the shared expert as row E
    int shared = 0;             // gfl_register_shared gave the layer a shared expert (row E) of bit widths shK
    int shK[3] = { 0, 0, 0 };
};

}  // namespace

struct gfl_ctx
{
    int device = 0;
    std::vector<Layer> layers;
    std::mutex mu;
    // decode workspace, reserved by gfl_register_layer for MAX_PICKS slots at the largest registered H and I and
    // carved with that fixed layout, so every call (and every graph captured from one) sees the same addresses
    void* ws = nullptr;
    size_t ws_bytes = 0;
    int ws_H = 0, ws_I = 0;
    int64_t calls = 0, picks = 0;
    // per-stage profiling events (gfl_profile_enable / gfl_profile_read)
    bool prof = false;
    std::vector<hipEvent_t> ev_pool;
    struct Rec { int stage; hipEvent_t a, b; };
    std::vector<Rec> recs;
    // silu(g) for every fp16 bit pattern g (the SwiGLU gate, see build_silu_table)
    float* silu_tab = nullptr;
    // slots per GEMV pass forced by GFL_SLOTS_PER_PASS (1, 2, 4 or 8; 0 = chosen from M)
    int ns_override = 0;
    // relay widths of the one-slot-per-pass EXACT launches forced by GFL_RELAY="g,d" (gate|up, down; 1, 2 or 4), or
    // "0" for the per-slot launches without relay; -1 = chosen from the call's size
    int rw_override[2] = { -1, -1 };
    // progress priority of the relay launches forced by GFL_RELAY_PRIO="g,d" (gate|up, down; 0 or 1); -1 = chosen
    // from the launch's waves per SIMD
    int prio_override[2] = { -1, -1 };
    // other GPU work runs beside this context's decode calls (gfl_ctx_set_shared): keep calls of 769..1536 gate|up
    // tile columns on the per-slot launches and run calls of up to 768 with 2 waves per column, which leave SIMDs free
    int shared = 0;
    // workspace of the prefill path (gfl_grouped_forward / gfl_grouped_reserve), grown on demand outside captures
    void* gws = nullptr;
    size_t gws_bytes = 0;
    // superseded workspaces: a graph captured before a workspace grew still holds their addresses, so they stay
    // allocated until gfl_ctx_destroy
    std::vector<void*> retired;
    // device memory allocated once by gfl_ctx_create: the status words (gfl::GFL_STATUS_*, sticky until
    // gfl_ctx_check), then the device worker's job state and its picks in selection form (gfl_ingress_serve)
    void* aux = nullptr;
    int* status = nullptr;           // [GFL_STATUS_WORDS]
    int64_t* ing_state = nullptr;    // [4] {job pending and accepted, its sequence number, 0, 0}
    int64_t* ing_sel = nullptr;      // [MAX_PICKS]
    float* ing_w = nullptr;          // [MAX_PICKS]
    // polls of a relay turn wait (GFL_RELAY_SPIN_LIMIT overrides it; 0 makes every wait expire, for tests)
    int spin_max = gfl::RELAY_SPIN_DEFAULT;
};

namespace {

struct Workspace
{
    gfl::PlanView pv;
    float* ygu;      // [2][2][cap][I]: [0] the gate|up outputs (EXACT), [1] the upper halves' partial sums (MFMA)
    uint16_t* xtd;   // [cap][I]
    float* yd;       // [cap][H]
    int* act_cnt;    // [cap][I/128] last-one counters of the SwiGLU stage (zero between calls)
    int* out_cnt;    // [cap][H/128] last-one counters of the combine (zero between calls)
    int* blk_cnt;    // [cap][H/128] half-block counters of the one-slot-per-pass down launch (zero between calls)
};

constexpr size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Decode workspace sizes for cap slots at hidden H and intermediate I: plan ints and the [cap][2] address table,
// gate|up outputs, down inputs, expert outputs, and the counter region (a tail of its own).
struct WsSizes
{
    size_t ints = 0, ygu = 0, xtd = 0, yd = 0, cnt = 0;
    constexpr size_t data() const { return ints + ygu + xtd + yd; }
};

constexpr WsSizes ws_sizes(int cap, int H, int I)
{
    WsSizes z;
    z.ints = align256(sizeof(int) * (size_t)(4 + 9 * cap + 4) + sizeof(uint64_t) * 2 * (size_t)cap);
    z.ygu = align256(sizeof(float) * 4 * (size_t)cap * I);
    z.xtd = align256(sizeof(uint16_t) * (size_t)cap * I);
    z.yd = align256(sizeof(float) * (size_t)cap * H);
    z.cnt = align256(sizeof(int) * (size_t)cap * (I / 128 + 2 * (H / 128)) * gfl::CNT_STRIDE);
    return z;
}

// Make the decode workspace hold MAX_PICKS slots at hidden H and intermediate I (and at every size reserved before).
// A larger buffer replaces the old one, which is retired, not freed: a graph captured earlier keeps valid addresses.
// The counter region is zeroed once here; the kernels leave every counter at zero when they finish.
int reserve_ws(gfl_ctx* c, int H, int I)
{
    const int nH = std::max(H, c->ws_H), nI = std::max(I, c->ws_I);
    if (c->ws && nH == c->ws_H && nI == c->ws_I) return GFL_OK;
    const WsSizes z = ws_sizes(gfl::MAX_PICKS, nH, nI);
    const size_t need = z.data() + z.cnt;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, need);
    if (e != hipSuccess) return fail(GFL_ENOMEM, std::string("workspace hipMalloc: ") + hipGetErrorString(e));
    e = hipMemset(p, 0, need);
    if (e != hipSuccess)
    {
        hipFree(p);
        return hip_fail(e, "workspace hipMemset");
    }
    if (c->ws) c->retired.push_back(c->ws);
    c->ws = p;
    c->ws_bytes = need;
    c->ws_H = nH;
    c->ws_I = nI;
    return GFL_OK;
}

// The fixed layout of a decode workspace at b laid out for cap slots at hidden wH and intermediate wI, with strides
// for a layer of hidden H and intermediate I (<= wH, wI): the addresses do not depend on the call's size.
void carve_at(void* base, int cap, int wH, int wI, int H, int I, Workspace& w)
{
    const WsSizes z = ws_sizes(cap, wH, wI);
    char* b = static_cast<char*>(base);
    int* ip = reinterpret_cast<int*>(b);
    w.pv.hdr = ip;
    w.pv.uexp = ip + 4;
    w.pv.uoff = w.pv.uexp + cap;
    w.pv.slot_pick = w.pv.uoff + cap + 1;
    w.pv.slot_u = w.pv.slot_pick + cap;
    w.pv.pick_slot = w.pv.slot_u + cap;
    w.pv.pick_job = w.pv.pick_slot + cap;
    w.pv.tok_slot = w.pv.pick_job + cap;
    w.pv.tok_w = reinterpret_cast<float*>(w.pv.tok_slot + cap);
    w.pv.tok_npk = reinterpret_cast<int*>(w.pv.tok_w + cap);
    w.pv.uptr = reinterpret_cast<uint64_t*>(ip + ((4 + 9 * (size_t)cap + 2 + 1) & ~size_t(1)));
    w.pv.cap_slots = cap;
    w.ygu = reinterpret_cast<float*>(b + z.ints);
    w.xtd = reinterpret_cast<uint16_t*>(b + z.ints + z.ygu);
    w.yd = reinterpret_cast<float*>(b + z.ints + z.ygu + z.xtd);
    w.act_cnt = reinterpret_cast<int*>(b + z.data());
    w.out_cnt = w.act_cnt + (size_t)cap * (I / 128) * gfl::CNT_STRIDE;
    w.blk_cnt = w.out_cnt + (size_t)cap * (H / 128) * gfl::CNT_STRIDE;
}

// the context's reserved workspace: MAX_PICKS slots at the largest registered H and I
void carve_ws(gfl_ctx* c, int H, int I, Workspace& w)
{
    carve_at(c->ws, gfl::MAX_PICKS, c->ws_H, c->ws_I, H, I, w);
}

bool k_ok(int K) { return K >= 2 && K <= 5; }

hipEvent_t take_event(gfl_ctx* c)
{
    if (!c->ev_pool.empty())
    {
        hipEvent_t e = c->ev_pool.back();
        c->ev_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

hipEvent_t take_event_cb(void* owner) { return take_event(static_cast<gfl_ctx*>(owner)); }

// runs `launch` with its kernels timed when profiling is on: launchers that take the kernel timer record each kernel's
// execution (start/stop events on its own dispatch); a stage whose launchers do not is bracketed by a pair of events
template <class F>
int staged(gfl_ctx* c, int stage, hipStream_t st, F&& launch)
{
    if (!c->prof) return launch();
    hipEvent_t a = take_event(c), b = take_event(c);
    if (!a || !b) return fail(GFL_ERUNTIME, "profiling: hipEventCreate failed");
    gfl::KernelTimer kt{ take_event_cb, c, {} };
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
    GFL_HIP(hipEventRecord(a, st));
    if (!capturing) gfl::g_kernel_timer = &kt;
    const int r = launch();
    gfl::g_kernel_timer = nullptr;
    GFL_HIP(hipEventRecord(b, st));
    if (kt.pairs.empty())
        c->recs.push_back({ stage, a, b });
    else
    {
        for (auto& pr : kt.pairs) c->recs.push_back({ stage, pr.first, pr.second });
        c->ev_pool.push_back(a);
        c->ev_pool.push_back(b);
    }
    return r;
}

// Argument checks shared by the decode forward entry points (returns GFL_OK or the failure code, message set).
int check_forward(gfl_ctx* c, int li, const uint16_t* x, const int64_t* sel, const void* w, int M, int topk,
                  const float* out, int mode, float act_limit, const char* who, int max_picks)
{
    const std::string f(who);
    if (!c) return fail(GFL_EINVAL, f + ": NULL argument");
    if (li < 0 || li >= (int)c->layers.size() || !c->layers[li].dptrs)
        return fail(GFL_EINVAL, f + ": layer not registered");
    // AFFINE (0) and I16 (2) name the reference CPU engine's speed modes; the device computes EXACT for them, which
    // lies closer to the fp64 expert than either of them does
    if (mode < GFL_MODE_AUTO || mode > GFL_MODE_MFMA)
        return fail(GFL_EINVAL, f + ": mode must be -1 (auto), 0 (affine), 1 (exact), 2 (i16) or 3 (mfma)");
    if (M < 0 || topk < 0 || topk > gfl::MAX_TOPK || (int64_t)M * topk > max_picks)
        return fail(GFL_EINVAL, f + ": need M >= 0, 0 <= topk <= 16 and M*topk <= " + std::to_string(max_picks));
    if ((int64_t)M * topk > gfl::MAX_PICKS && mode == GFL_MODE_MFMA)
        return fail(GFL_EINVAL, f + ": mode MFMA takes M*topk <= 1024 (gfl_grouped_forward is the MFMA path for "
                                    "more)");
    if (!std::isfinite(act_limit) || act_limit < 0) return fail(GFL_EINVAL, f + ": act_limit must be >= 0");
    // an empty batch touches no buffer (they may be NULL); without picks only x and out are used
    if (M > 0 && (!x || !out || (topk > 0 && (!sel || !w)))) return fail(GFL_EINVAL, f + ": NULL argument");
    if (reinterpret_cast<uintptr_t>(x) & 15) return fail(GFL_EINVAL, f + ": x must be 16-byte aligned");
    return GFL_OK;
}

// The decode forward on workspace ws (caller holds c->mu, device set). prof: bracket the stages with the context's
// profiling events when profiling is on (the no-allocation entry point does not: event creation is left out of it).
// nsh = M: the layer's shared expert rides on the relay launches as one more pick per token (gfl_moe_forward_shared);
// a call that does not take them then returns GFL_EUNSUPPORTED before anything is launched.
int run_forward(gfl_ctx* c, const Layer& L, const Workspace& ws, const uint16_t* x, const int64_t* sel,
                const void* w, int w_is_half, int M, int topk, float* out, int mode, float act_limit, hipStream_t st,
                bool prof, int nsh = 0)
{
    const int P = M * topk;
    const int umax = P < L.E ? P : L.E;
    // slots per pass of the GEMV (its LDS holds NS transformed inputs). With one slot per pass the launches run a
    // workgroup per slot, so an expert picked by several tokens is streamed once per slot in parallel; with more,
    // a workgroup per union entry takes the entry's slots in passes. Measured on MI355X (config 1 uniform, config 2
    // Zipf, top-8 of 288): per slot is 5-15% faster at M = 2..4; two slots per pass are 4% faster at M = 16, 8% at
    // M = 32 and 16% at M = 64 (there the extra weight streams of per slot cost more than its smaller LDS footprint
    // gains). Four slots per pass match two at M = 64 and lose elsewhere; eight lose everywhere.
    //
    // Mode MFMA accumulates the GEMVs with MFMAs (same weights, transforms and rounding points; sums over the hidden
    // dimension in MFMA order) with a workgroup per union entry taking up to 4 of its slots per pass: an expert's
    // tiles are decoded once for all its tokens of the pass.
    const int mf = mode == GFL_MODE_MFMA ? 1 : 0;
    int ns = mf ? std::min(M, 4) : M <= 8 ? 1 : 2;
    if (c->ns_override > 0) ns = std::min(c->ns_override, mf ? std::min(M, 16) : M);
    // With one slot per pass the calls run the relay launches: a workgroup per (pick, tile columns), rw waves per
    // column, each streaming and decoding every rw-th group of 8 tile rows while the column's accumulators pass from
    // wave to wave in tile-row order (chain_relay). With one wave per column a call of few columns leaves most SIMDs
    // idle; rw waves per column put rw times the waves on the chip. Measured on MI355X (config-1 layers, 4 cycled):
    // one expert per call (192 gate|up columns) 39.2 -> 27.5 us with 4 waves per column; 8 picks (1,536 columns)
    // 58.4 -> 56.4 us with 2 waves per gate|up column and 1 per down column. From 16 picks on, one wave per column
    // beats the per-slot launches (gu_kernel / down_kernel) by 2-5% on uniform routing (us per token at M = 2, 3, 4, 6,
    // 8: 39.7 -> 38.8, 36.8 -> 35.1, 33.2 -> 31.6, 31.5 -> 30.1, 30.5 -> 29.5) and matches them on Zipf routing.
    // The relay launches at 8 picks fill every SIMD with 3 waves, so a shared expert on a side stream (k_overlap)
    // then waits (routed + shared 71.3 -> 79.1 us): a context told that other work runs beside it (gfl_ctx_set_shared)
    // keeps those calls on the per-slot launches. From 16 picks on the one-wave relay launches stay (routed + shared
    // at M = 4 overlapped: 43.2 us per token with the per-slot launches, 41.5 with them). A shared context's calls of
    // up to 768 columns (a shared expert beside a routed call that fills every SIMD) take 2 waves per gate|up column
    // and 1 per down column instead of 4: routed + shared at M = 4 overlapped 41.1 -> 38.8 us per token.
    int rw[2] = { 0, 0 };
    // the relay down launch forms each token's combine order from one pick per lane of a wave: at most 64 picks
    if (!mf && ns == 1 && P <= 64)
    {
        const int64_t cgu = (int64_t)(P + nsh) * 2 * (L.I / 16), cdn = (int64_t)(P + nsh) * (L.H / 16);   // columns
        if (cgu <= 768 && c->shared)
        {
            rw[0] = 2;
            rw[1] = 1;
        }
        else if (cgu <= 768)
        {
            rw[0] = 4;
            rw[1] = cdn <= 768 ? 4 : cdn <= 1536 ? 2 : 1;
        }
        else if (cgu > 1536)
        {
            rw[0] = 1;
            rw[1] = 1;
        }
        else if (!c->shared)
        {
            rw[0] = 2;
            rw[1] = 1;
        }
        if (c->rw_override[0] >= 0) { rw[0] = c->rw_override[0]; rw[1] = c->rw_override[1]; }
    }
    // progress priority of the relay launches: -1 = chosen by each launch from its waves per SIMD
    const int prio[2] = { c->prio_override[0], c->prio_override[1] };
    if (nsh && !rw[0])
        return fail(GFL_EUNSUPPORTED, "gfl_moe_forward_shared: this call does not take the relay launches (more than 64 "
                                      "picks, mode MFMA, or a context set shared at 769..1536 columns)");
    // above 64 picks the launches without relay take the routing plan from a launch of its own (plan_kernel) instead
    // of every workgroup building it in LDS. Measured on MI355X (config 1, us per token): M = 32 25.9 -> 24.5, M = 64
    // 23.3 -> 21.5, and with the plan launch at 9-12 us, M = 12..24 0.1-0.4 faster than building it per workgroup.
    // Up to 64 picks a workgroup builds it from one wave's registers (build_plan_wave), cheaper than a launch.
    const int gplan = !rw[0] && P > 64 ? 1 : 0;
    if (gfl::gate_up_lds_bytes(L.K[0], ns, L.H, P, L.E, mf, rw[0], gplan) > gfl::LDS_LIMIT ||
        gfl::gate_up_lds_bytes(L.K[1], ns, L.H, P, L.E, mf, rw[0], gplan) > gfl::LDS_LIMIT ||
        gfl::down_lds_bytes(L.K[2], ns, L.I, P, L.E, mf, rw[1]) > gfl::LDS_LIMIT)
        return fail(GFL_EINVAL, "gfl_moe_forward: shape needs more than 160 KB of LDS per workgroup");
    const int wh = w_is_half ? 1 : 0;
    auto gate_up = [&] {
        if (L.K[0] == L.K[1])
            return gfl::launch_gate_up(L.K[0], ns, L.dptrs, 0, 2, sel, w, wh, P, topk, L.E, L.H, L.I, umax, x, ws.ygu,
                                       ws.xtd, ws.act_cnt, c->silu_tab, act_limit, ws.pv, out, mf, rw[0], prio[0], nsh, gplan,
                                       c->status, c->spin_max, st);
        if (gfl::launch_gate_up(L.K[0], ns, L.dptrs, 0, 1, sel, w, wh, P, topk, L.E, L.H, L.I, umax, x, ws.ygu,
                                ws.xtd, ws.act_cnt, c->silu_tab, act_limit, ws.pv, out, mf, rw[0], prio[0], nsh, gplan,
                                c->status, c->spin_max, st))
            return -1;
        return gfl::launch_gate_up(L.K[1], ns, L.dptrs, 1, 1, sel, w, wh, P, topk, L.E, L.H, L.I, umax, x, ws.ygu,
                                   ws.xtd, ws.act_cnt, c->silu_tab, act_limit, ws.pv, out, mf, rw[0], prio[0], nsh, gplan,
                                   c->status, c->spin_max, st);
    };
    auto down = [&] {
        return gfl::launch_down(L.K[2], ns, L.dptrs, topk, L.H, L.I, umax, P, L.E, sel, w, wh, ws.pv, ws.xtd, ws.yd,
                                ws.out_cnt, ws.blk_cnt, out, mf, rw[1], prio[1], nsh, c->status, c->spin_max, st);
    };
    int r = prof ? staged(c, 1, st, gate_up) : gate_up();
    if (!r) r = prof ? staged(c, 3, st, down) : down();
    if (r) return r > 0 ? r : fail(GFL_EINVAL, "gfl_moe_forward: unsupported K or launch shape");
    GFL_HIP(hipGetLastError());
    c->calls += 1;
    c->picks += P;
    return GFL_OK;
}

// ---------------------------------------------------------------------------------------------------------------
// Static scratch of gfl_moe_forward_noalloc: one decode workspace per device in a file-scope device array, laid out
// for GFL_NOALLOC_MAX_PICKS slots at GFL_NOALLOC_MAX_H x GFL_NOALLOC_MAX_I. Every device the library runs on holds
// its own copy until the process ends. The host-side name `scratch` is not a device address: its address on each
// device is taken once with hipGetSymbolAddress and only that pointer is handed to kernels.
// ---------------------------------------------------------------------------------------------------------------

constexpr WsSizes kScratch = ws_sizes(GFL_NOALLOC_MAX_PICKS, GFL_NOALLOC_MAX_H, GFL_NOALLOC_MAX_I);
constexpr size_t kScratchBytes = kScratch.data() + kScratch.cnt;
static_assert(kScratchBytes <= ((size_t)8 << 20), "the no-allocation scratch stays below 8 MiB");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// zeroes the counter region (a kernel rather than hipMemsetAsync, so a stream capture may record it)
__global__ void zero_words(int* p, size_t n)
{
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

// The result of a call without picks (topk = 0, as the reference's tier_forward returns for sel [m, 0]): M rows of
// zeros, written by a fill kernel (capture-safe, no allocation).
int forward_without_picks(gfl_ctx* c, const Layer& L, int M, float* out, hipStream_t st)
{
    GFL_HIP(hipSetDevice(c->device));
    hipLaunchKernelGGL(zero_words, dim3(64), dim3(256), 0, st, reinterpret_cast<int*>(out), (size_t)M * L.H);
    GFL_HIP(hipGetLastError());
    return GFL_OK;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
// per device: the last enqueued no-allocation call's completion. Every eager call waits for it on its own stream and
// records it again (under g_scratch_mu), so calls from different contexts and streams run one after another on the
// device's one array. Created by gfl_ctx_create, so the no-allocation calls create nothing.
hipEvent_t g_scratch_ev[kMaxDevices] = {};

int scratch_event_for_device(int device)
{
    if (device < 0 || device >= kMaxDevices) return GFL_OK;   // gfl_moe_forward_noalloc refuses such a device
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_ev[device]) GFL_HIP(hipEventCreateWithFlags(&g_scratch_ev[device], hipEventDisableTiming));
    return GFL_OK;
}

// This device's scratch address (device current, g_scratch_mu held). On the first call for the device: look the
// address up and clear the counter region on `st` (the kernels leave every counter at zero when they finish, so once
// is enough).
int scratch_for_device(int device, hipStream_t st, void** out)
{
    if (device < 0 || device >= kMaxDevices) return fail(GFL_EINVAL, "gfl_moe_forward_noalloc: device index too large");
    if (!g_scratch_ptr[device])
    {
        void* p = nullptr;
        GFL_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(GFL_ERUNTIME, "gfl_moe_forward_noalloc: hipGetSymbolAddress returned NULL");
        const size_t nw = kScratch.cnt / sizeof(int);
        hipLaunchKernelGGL(zero_words, dim3(64), dim3(256), 0, st, reinterpret_cast<int*>(static_cast<char*>(p) +
                                                                                         kScratch.data()), nw);
        GFL_HIP(hipGetLastError());
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return GFL_OK;
}

}  // namespace

extern "C" {

const char* gfl_last_error(void) { return g_err.c_str(); }

int gfl_version(void) { return 101; }

// The SwiGLU gate of the reference is silu(g) = g / (1 + std::exp(-g)) in fp32 (ft_core.h:123), i.e. the host C
// library's expf. g is always fp16-valued (out_block rounds it, ft_core.h:109), so the exponential the device needs
// is expf over the 65,536 fp16 bit patterns. glibc's expf is not correctly rounded on every one of them (it is
// within 0.502 ulp), so no device formula reproduces it exactly; the table is evaluated here, by the same library
// call the reference makes, and the device table of silu (build_silu_table) is formed from it.
static void build_exp_table(float* tab)
{
    for (uint32_t b = 0; b < 65536; ++b)
    {
        const uint16_t bits = (uint16_t)b;
        _Float16 h;
        std::memcpy(&h, &bits, 2);
        const float g = (float)h;     // exact
        tab[b] = std::exp(-g);
    }
}

// silu(g) = g / (1 + expf(-g)) as the reference evaluates it in fp32 (ft_core.h:123): the library expf, then one
// fp32 add and one fp32 division, each rounded. As g is fp16-valued, the whole gate is a function of g's 16 bits and
// the activation kernels look it up instead of dividing.
static void build_silu_table(float* tab)
{
    build_exp_table(tab);
    for (uint32_t b = 0; b < 65536; ++b)
    {
        const uint16_t bits = (uint16_t)b;
        _Float16 h;
        std::memcpy(&h, &bits, 2);
        const float g = (float)h;
        const float d = 1.0f + tab[b];
        tab[b] = g / d;
    }
}

int gfl_exp_table(float* out, int n)
{
    if (!out || n < 65536) return fail(GFL_EINVAL, "gfl_exp_table: needs a host array of 65536 floats");
    build_exp_table(out);
    return GFL_OK;
}

int gfl_silu_table(float* out, int n)
{
    if (!out || n < 65536) return fail(GFL_EINVAL, "gfl_silu_table: needs a host array of 65536 floats");
    build_silu_table(out);
    return GFL_OK;
}

int gfl_ctx_create(int device, gfl_ctx** out)
{
    if (!out) return fail(GFL_EINVAL, "gfl_ctx_create: out is NULL");
    int n = 0;
    GFL_HIP(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(GFL_EINVAL, "gfl_ctx_create: no such device");
    GFL_HIP(hipSetDevice(device));
    std::vector<float> tab(65536);
    build_silu_table(tab.data());
    float* dtab = nullptr;
    if (hipMalloc(&dtab, tab.size() * sizeof(float)) != hipSuccess)
        return fail(GFL_ENOMEM, "gfl_ctx_create: silu table");
    const hipError_t e = hipMemcpy(dtab, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess)
    {
        hipFree(dtab);
        return fail(GFL_ERUNTIME, std::string("gfl_ctx_create: ") + hipGetErrorString(e));
    }
    // status words, the device worker's job state and picks: one allocation, zeroed
    const size_t aux_bytes = 256 + 256 + sizeof(int64_t) * gfl::MAX_PICKS + sizeof(float) * gfl::MAX_PICKS;
    void* aux = nullptr;
    if (hipMalloc(&aux, aux_bytes) != hipSuccess)
    {
        hipFree(dtab);
        return fail(GFL_ENOMEM, "gfl_ctx_create: status words");
    }
    if (hipMemset(aux, 0, aux_bytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
    {
        hipFree(aux);
        hipFree(dtab);
        return fail(GFL_ERUNTIME, "gfl_ctx_create: clearing the status words failed");
    }
    gfl_ctx* c = new gfl_ctx();
    c->device = device;
    c->silu_tab = dtab;
    c->aux = aux;
    c->status = static_cast<int*>(aux);
    c->ing_state = reinterpret_cast<int64_t*>(static_cast<char*>(aux) + 256);
    c->ing_sel = reinterpret_cast<int64_t*>(static_cast<char*>(aux) + 512);
    c->ing_w = reinterpret_cast<float*>(c->ing_sel + gfl::MAX_PICKS);
    if (const int r = scratch_event_for_device(device))
    {
        hipFree(aux);
        hipFree(dtab);
        delete c;
        return r;
    }
    if (const char* e = std::getenv("GFL_RELAY_SPIN_LIMIT"))
    {
        const long v = std::atol(e);
        if (v >= 0 && v <= gfl::RELAY_SPIN_DEFAULT) c->spin_max = (int)v;
    }
    if (const char* e = std::getenv("GFL_SLOTS_PER_PASS"))
    {
        const int v = std::atoi(e);
        if (v == 1 || v == 2 || v == 4 || v == 8) c->ns_override = v;
    }
    if (const char* e = std::getenv("GFL_RELAY"))
    {
        int g = -1, d = -1;
        const int n = std::sscanf(e, "%d,%d", &g, &d);
        auto ok = [](int v) { return v == 0 || v == 1 || v == 2 || v == 4; };
        if (n == 1 && g == 0) c->rw_override[0] = c->rw_override[1] = 0;
        else if (n == 2 && ok(g) && ok(d) && g > 0 && d > 0) { c->rw_override[0] = g; c->rw_override[1] = d; }
    }
    if (const char* e = std::getenv("GFL_RELAY_PRIO"))
    {
        int g = -1, d = -1;
        if (std::sscanf(e, "%d,%d", &g, &d) == 2 && (g == 0 || g == 1) && (d == 0 || d == 1))
        {
            c->prio_override[0] = g;
            c->prio_override[1] = d;
        }
    }

    *out = c;
    return GFL_OK;
}

int gfl_ctx_destroy(gfl_ctx* c)
{
    if (!c) return GFL_OK;
    hipSetDevice(c->device);
    for (auto& r : c->recs) { hipEventDestroy(r.a); hipEventDestroy(r.b); }
    for (auto e : c->ev_pool) hipEventDestroy(e);
    for (auto& L : c->layers)
        if (L.dptrs) hipFree(L.dptrs);
    if (c->ws) hipFree(c->ws);
    if (c->gws) hipFree(c->gws);
    for (void* p : c->retired) hipFree(p);
    if (c->silu_tab) hipFree(c->silu_tab);
    if (c->aux) hipFree(c->aux);
    delete c;
    return GFL_OK;
}

int gfl_register_layer(gfl_ctx* c, int li, int E, int H, int I, int k_gate, int k_up, int k_down, const uint64_t* ptrs)
{
    if (!c || !ptrs) return fail(GFL_EINVAL, "gfl_register_layer: NULL argument");
    if (li < 0 || li > 4096) return fail(GFL_EINVAL, "gfl_register_layer: layer index out of range");
    if (E < 1 || E > gfl::MAX_EXPERTS) return fail(GFL_EINVAL, "gfl_register_layer: E must be 1..1024");
    if (H < 256 || I < 256 || H % 256 || I % 256 || H > GFL_MAX_DIM || I > GFL_MAX_DIM)
        return fail(GFL_EINVAL, "gfl_register_layer: H and I must be multiples of 256 up to " +
                                    std::to_string(GFL_MAX_DIM));
    if (!k_ok(k_gate) || !k_ok(k_up) || !k_ok(k_down)) return fail(GFL_EINVAL, "gfl_register_layer: K must be 2..5");
    // trellis words are read 4 bytes at a time, suh/svh 16 bytes at a time
    for (int i = 0; i < E * 9; ++i)
        if (ptrs[i] == 0 || (ptrs[i] & (i % 9 < 3 ? 3 : 15)))
            return fail(GFL_EINVAL, "gfl_register_layer: NULL or misaligned device pointer (trellis 4-byte, suh/svh "
                                    "16-byte alignment)");
    std::lock_guard<std::mutex> g(c->mu);
    GFL_HIP(hipSetDevice(c->device));
    if ((int)c->layers.size() <= li) c->layers.resize(li + 1);
    Layer& L = c->layers[li];
    if (L.dptrs) GFL_HIP(hipFree(L.dptrs));
    L.dptrs = nullptr;
    GFL_HIP(hipMalloc(&L.dptrs, sizeof(uint64_t) * 9 * (size_t)E));
    GFL_HIP(hipMemcpy(L.dptrs, ptrs, sizeof(uint64_t) * 9 * (size_t)E, hipMemcpyHostToDevice));
    L.E = E; L.H = H; L.I = I; L.K[0] = k_gate; L.K[1] = k_up; L.K[2] = k_down;
    L.shared = 0;
    // the decode workspace for this shape, reserved now so that no forward call allocates
    return reserve_ws(c, H, I);
}

int gfl_register_shared(gfl_ctx* c, int li, int k_gate, int k_up, int k_down, const uint64_t* ptr_row)
{
    if (!c || !ptr_row) return fail(GFL_EINVAL, "gfl_register_shared: NULL argument");
    if (li < 0 || li >= (int)c->layers.size() || !c->layers[li].dptrs)
        return fail(GFL_EINVAL, "gfl_register_shared: layer not registered");
    if (!k_ok(k_gate) || !k_ok(k_up) || !k_ok(k_down)) return fail(GFL_EINVAL, "gfl_register_shared: K must be 2..5");
    for (int i = 0; i < 9; ++i)
        if (ptr_row[i] == 0 || (ptr_row[i] & (i < 3 ? 3 : 15)))
            return fail(GFL_EINVAL, "gfl_register_shared: NULL or misaligned device pointer (trellis 4-byte, suh/svh "
                                    "16-byte alignment)");
    std::lock_guard<std::mutex> g(c->mu);
    GFL_HIP(hipSetDevice(c->device));
    Layer& L = c->layers[li];
    // the routed table with the shared expert as row E
    uint64_t* t = nullptr;
    GFL_HIP(hipMalloc(&t, sizeof(uint64_t) * 9 * (size_t)(L.E + 1)));
    hipError_t e = hipMemcpy(t, L.dptrs, sizeof(uint64_t) * 9 * (size_t)L.E, hipMemcpyDeviceToDevice);
    if (e == hipSuccess) e = hipMemcpy(t + 9 * (size_t)L.E, ptr_row, sizeof(uint64_t) * 9, hipMemcpyHostToDevice);
    if (e != hipSuccess)
    {
        hipFree(t);
        return hip_fail(e, "gfl_register_shared");
    }
    GFL_HIP(hipFree(L.dptrs));
    L.dptrs = t;
    L.shared = 1;
    L.shK[0] = k_gate; L.shK[1] = k_up; L.shK[2] = k_down;
    return GFL_OK;
}

static int run_forward_grouped_plan(gfl_ctx* c, const Layer& L, const uint16_t* x, const int64_t* sel, const void* w,
                                    int w_is_half, int M, int topk, float* out, float act_limit, hipStream_t st);

int gfl_moe_forward(gfl_ctx* c, int li, const uint16_t* x, const int64_t* sel, const void* w, int w_is_half, int M,
                    int topk, float* out, int mode, float act_limit, gfl_stream stream)
{
    if (const int r = check_forward(c, li, x, sel, w, M, topk, out, mode, act_limit, "gfl_moe_forward",
                                    gfl::MAX_GROUPED_PICKS))
        return r;
    if (M == 0) return GFL_OK;   // an empty batch: nothing to compute
    std::lock_guard<std::mutex> g(c->mu);
    const Layer& L = c->layers[li];
    if (topk == 0) return forward_without_picks(c, L, M, out, reinterpret_cast<hipStream_t>(stream));
    GFL_HIP(hipSetDevice(c->device));
    if (M * topk > gfl::MAX_PICKS)
        return run_forward_grouped_plan(c, L, x, sel, w, w_is_half, M, topk, out, act_limit,
                                        reinterpret_cast<hipStream_t>(stream));
    if (!c->ws || L.H > c->ws_H || L.I > c->ws_I) return fail(GFL_ERUNTIME, "gfl_moe_forward: workspace not reserved");
    Workspace ws;
    carve_ws(c, L.H, L.I, ws);
    return run_forward(c, L, ws, x, sel, w, w_is_half, M, topk, out, mode, act_limit,
                       reinterpret_cast<hipStream_t>(stream), true);
}

int gfl_moe_forward_shared(gfl_ctx* c, int li, const uint16_t* x, const int64_t* sel, const void* w, int w_is_half,
                           int M, int topk, float* out, int mode, float act_limit, gfl_stream stream)
{
    const char* who = "gfl_moe_forward_shared";
    if (const int r = check_forward(c, li, x, sel, w, M, topk, out, mode, act_limit, who, gfl::MAX_GROUPED_PICKS))
        return r;
    std::lock_guard<std::mutex> g(c->mu);
    const Layer& L = c->layers[li];
    if (!L.shared) return fail(GFL_EINVAL, std::string(who) + ": the layer has no shared expert (gfl_register_shared)");
    if (M == 0) return GFL_OK;   // an empty batch: nothing to compute
    // the shared expert's picks run in the routed launches' kernels, instantiated for the layer's bit widths
    if (topk == 0 || L.shK[0] != L.K[0] || L.shK[1] != L.K[1] || L.shK[2] != L.K[2] || (int64_t)M * (topk + 1) >
        gfl::MAX_PICKS)
        return fail(GFL_EUNSUPPORTED, std::string(who) + ": needs topk >= 1, M*(topk+1) <= 1024 and the shared "
                                                         "expert's bit widths equal to the layer's");
    GFL_HIP(hipSetDevice(c->device));
    if (!c->ws || L.H > c->ws_H || L.I > c->ws_I) return fail(GFL_ERUNTIME, std::string(who) + ": workspace not reserved");
    Workspace ws;
    carve_ws(c, L.H, L.I, ws);
    return run_forward(c, L, ws, x, sel, w, w_is_half, M, topk, out, mode, act_limit,
                       reinterpret_cast<hipStream_t>(stream), true, M);
}

int gfl_moe_forward_noalloc(gfl_ctx* c, int li, const uint16_t* x, const int64_t* sel, const void* w, int w_is_half,
                            int M, int topk, float* out, int mode, float act_limit, gfl_stream stream)
{
    const char* who = "gfl_moe_forward_noalloc";
    if (const int r = check_forward(c, li, x, sel, w, M, topk, out, mode, act_limit, who, GFL_NOALLOC_MAX_PICKS))
        return r;
    if (M == 0) return GFL_OK;   // an empty batch: nothing to compute
    std::lock_guard<std::mutex> g(c->mu);
    const Layer& L = c->layers[li];
    if (topk == 0) return forward_without_picks(c, L, M, out, reinterpret_cast<hipStream_t>(stream));
    if ((int64_t)M * topk > GFL_NOALLOC_MAX_PICKS || L.H > GFL_NOALLOC_MAX_H || L.I > GFL_NOALLOC_MAX_I)
        return fail(GFL_EINVAL, std::string(who) + ": needs M*topk <= " + std::to_string(GFL_NOALLOC_MAX_PICKS) +
                                    ", H <= " + std::to_string(GFL_NOALLOC_MAX_H) + " and I <= " +
                                    std::to_string(GFL_NOALLOC_MAX_I) + " (the static scratch array's layout)");
    GFL_HIP(hipSetDevice(c->device));
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    std::lock_guard<std::mutex> gs(g_scratch_mu);
    void* base = nullptr;
    if (const int r = scratch_for_device(c->device, st, &base)) return r;
    hipEvent_t ev = g_scratch_ev[c->device];
    if (!ev) return fail(GFL_ERUNTIME, std::string(who) + ": no ordering event for this device");
    // eager calls are ordered through the device's event; a captured call is ordered only within its graph (its
    // replays must not overlap other calls on the device)
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
    if (!capturing) GFL_HIP(hipStreamWaitEvent(st, ev, 0));
    Workspace ws;
    carve_at(base, GFL_NOALLOC_MAX_PICKS, GFL_NOALLOC_MAX_H, GFL_NOALLOC_MAX_I, L.H, L.I, ws);
    const int r = run_forward(c, L, ws, x, sel, w, w_is_half, M, topk, out, mode, act_limit, st, false);
    if (!capturing) GFL_HIP(hipEventRecord(ev, st));
    return r;
}

// The prefill workspace of a context, grown on demand (never inside a graph capture). Layout: the grouped plan's ints,
// then one data region for whichever path runs: the MFMA grouped path's xt [2][P][H], ygu [2][P][I], xd [P][I],
// yraw [P][H] (fp16), or the EXACT chains' xte [2][P][H] fp32, ygue [2][P][I] fp16, xde [P][I] fp32, yre [P][H] fp16.
struct Gws
{
    gfl::GPlan gp;
    uint16_t *xt, *ygu16, *xd, *yraw;
    float *xte, *xde;
    uint16_t *ygue, *yre;
};

static int grow(gfl_ctx* c, hipStream_t st, void** buf, size_t* have, size_t need, bool zero, const char* who)
{
    if (need <= *have) return GFL_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (st && hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
        return fail(GFL_EINVAL, std::string(who) + ": the workspace must be sized before graph capture "
                                                  "(gfl_grouped_reserve, or one call of this shape first)");
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, need);
    if (e != hipSuccess) return fail(GFL_ENOMEM, std::string(who) + ": workspace hipMalloc: " + hipGetErrorString(e));
    if (zero && (e = hipMemset(p, 0, need)) != hipSuccess)
    {
        hipFree(p);
        return hip_fail(e, "workspace hipMemset");
    }
    // the old buffer is retired, not freed: a graph captured before this growth still holds its addresses
    if (*buf) c->retired.push_back(*buf);
    *buf = p;
    *have = need;
    return GFL_OK;
}

static int grouped_workspace(gfl_ctx* c, hipStream_t st, int P, int M, int E, int H, int I, const char* who, Gws& w)
{
    const size_t nch = (P + gfl::GP_PLAN_CHUNK - 1) / gfl::GP_PLAN_CHUNK;
    const size_t n_int = 4 + (size_t)E + (E + 1) + 7 * (size_t)P + (size_t)M + (size_t)P + (size_t)E + nch * (E + 1);
    const size_t b_int = align256(sizeof(int) * n_int);
    const size_t g_xt = align256(2 * 2 * (size_t)P * H), g_ygu = align256(2 * 2 * (size_t)P * I);
    const size_t g_xd = align256(2 * (size_t)P * I), g_yr = align256(2 * (size_t)P * H);
    const size_t c_xt = align256(4 * 2 * (size_t)P * H), c_ygu = align256(2 * 2 * (size_t)P * I);
    const size_t c_xd = align256(4 * (size_t)P * I), c_yr = align256(2 * (size_t)P * H);
    const size_t data = std::max(g_xt + g_ygu + g_xd + g_yr, c_xt + c_ygu + c_xd + c_yr);
    if (const int r = grow(c, st, &c->gws, &c->gws_bytes, b_int + data, false, who)) return r;
    char* b = static_cast<char*>(c->gws);
    int* ip = reinterpret_cast<int*>(b);
    gfl::GPlan& gp = w.gp;
    gp.hdr = ip;
    gp.cnt = gp.hdr + 4;
    gp.off = gp.cnt + E;
    gp.slot_pick = gp.off + E + 1;
    gp.slot_e = gp.slot_pick + P;
    gp.pick_slot = gp.slot_e + P;
    gp.pick_c = gp.pick_slot + P;
    gp.slot_job = gp.pick_c + P;
    gp.tok_slot = gp.slot_job + P;
    gp.tok_w = reinterpret_cast<float*>(gp.tok_slot + P);
    gp.tok_npk = reinterpret_cast<int*>(gp.tok_w + P);
    gp.eord = gp.tok_npk + M;
    gp.ccnt = gp.eord + E;
    char* d = b + b_int;
    w.xt = reinterpret_cast<uint16_t*>(d);
    w.ygu16 = reinterpret_cast<uint16_t*>(d + g_xt);
    w.xd = reinterpret_cast<uint16_t*>(d + g_xt + g_ygu);
    w.yraw = reinterpret_cast<uint16_t*>(d + g_xt + g_ygu + g_xd);
    w.xte = reinterpret_cast<float*>(d);
    w.ygue = reinterpret_cast<uint16_t*>(d + c_xt);
    w.xde = reinterpret_cast<float*>(d + c_xt + c_ygu);
    w.yre = reinterpret_cast<uint16_t*>(d + c_xt + c_ygu + c_xd);
    return GFL_OK;
}

// EXACT above MAX_PICKS picks (caller holds c->mu, device set): the grouped plan of the prefill path, then the
// reference's accumulator chains with each weight decoded once per pass of up to 64 of an expert's slots
// (launch_exact_chains, bit-identical to the decode path).
static int run_forward_grouped_plan(gfl_ctx* c, const Layer& L, const uint16_t* x, const int64_t* sel, const void* w,
                                    int w_is_half, int M, int topk, float* out, float act_limit, hipStream_t st)
{
    const int P = M * topk;
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) & 15)
        return fail(GFL_EINVAL, "gfl_moe_forward: above 1024 picks x and out must be 16-byte aligned");
    if ((size_t)P * (size_t)std::max(L.H, L.I) * 4 > (size_t)0x7fffffff)
        return fail(GFL_EINVAL, "gfl_moe_forward: M*topk*max(H, I) must stay below 2^29 above 1024 picks");
    Gws ws;
    if (const int rc = grouped_workspace(c, st, P, M, L.E, L.H, L.I, "gfl_moe_forward", ws)) return rc;
    const int r = staged(c, 1, st, [&] {
        return gfl::launch_exact_chains(L.dptrs, sel, w, w_is_half ? 1 : 0, P, topk, L.E, L.H, L.I, L.K[0], L.K[1],
                                        L.K[2], x, ws.gp, P, ws.xte, ws.ygue, ws.xde, ws.yre, c->silu_tab, act_limit,
                                        out, st);
    });
    if (r) return r > 0 ? r : fail(GFL_EINVAL, "gfl_moe_forward: unsupported K or launch shape");
    GFL_HIP(hipGetLastError());
    c->calls += 1;
    c->picks += P;
    return GFL_OK;
}

int gfl_grouped_forward(gfl_ctx* c, int li, const uint16_t* x, const int64_t* sel, const void* w, int w_is_half,
                        int M, int topk, float* out, float act_limit, gfl_stream stream)
{
    if (!c) return fail(GFL_EINVAL, "gfl_grouped_forward: NULL argument");
    if (li < 0 || li >= (int)c->layers.size() || !c->layers[li].dptrs)
        return fail(GFL_EINVAL, "gfl_grouped_forward: layer not registered");
    if (M < 0 || topk < 0 || topk > gfl::MAX_TOPK || (int64_t)M * topk > gfl::MAX_GROUPED_PICKS)
        return fail(GFL_EINVAL, "gfl_grouped_forward: need M >= 0, 0 <= topk <= 16 and M*topk <= 65536");
    if (!std::isfinite(act_limit) || act_limit < 0)
        return fail(GFL_EINVAL, "gfl_grouped_forward: act_limit must be >= 0");
    if (M == 0) return GFL_OK;   // an empty batch: nothing to compute (its buffers may be NULL)
    if (!x || !out || (topk > 0 && (!sel || !w))) return fail(GFL_EINVAL, "gfl_grouped_forward: NULL argument");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) & 15)
        return fail(GFL_EINVAL, "gfl_grouped_forward: x and out must be 16-byte aligned");
    std::lock_guard<std::mutex> g(c->mu);
    const Layer& L = c->layers[li];
    if (topk == 0) return forward_without_picks(c, L, M, out, reinterpret_cast<hipStream_t>(stream));
    if (L.H % 256 || L.I % 256) return fail(GFL_EINVAL, "gfl_grouped_forward: H and I must be multiples of 256");
    // the GEMMs address their fp16 inputs [picks][max(H, I)] through 32-bit buffer offsets
    if ((size_t)M * topk * (size_t)std::max(L.H, L.I) * 2 > (size_t)0x7fffffff)
        return fail(GFL_EINVAL, "gfl_grouped_forward: M*topk*max(H, I) must stay below 2^30");
    GFL_HIP(hipSetDevice(c->device));
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int P = M * topk, E = L.E, H = L.H, I = L.I;
    Gws ws;
    if (const int rc = grouped_workspace(c, st, P, M, E, H, I, "gfl_grouped_forward", ws)) return rc;
    const int r = staged(c, 2, st, [&] {
        return gfl::launch_grouped(L.dptrs, sel, w, w_is_half ? 1 : 0, P, topk, E, H, I, L.K[0], L.K[1], L.K[2], x,
                                   ws.gp, P, ws.xt, ws.ygu16, ws.xd, ws.yraw, c->silu_tab, act_limit, out, st);
    });
    if (r) return fail(GFL_ERUNTIME, "gfl_grouped_forward: launch set-up failed");
    GFL_HIP(hipGetLastError());
    c->calls += 1;
    c->picks += P;
    return GFL_OK;
}

int gfl_grouped_reserve(gfl_ctx* c, int max_picks)
{
    if (!c) return fail(GFL_EINVAL, "gfl_grouped_reserve: NULL context");
    if (max_picks < 1 || max_picks > gfl::MAX_GROUPED_PICKS)
        return fail(GFL_EINVAL, "gfl_grouped_reserve: need 1 <= max_picks <= 65536");
    std::lock_guard<std::mutex> g(c->mu);
    int E = 0, H = 0, I = 0;
    for (const auto& L : c->layers)
        if (L.dptrs) { E = std::max(E, L.E); H = std::max(H, L.H); I = std::max(I, L.I); }
    if (!E) return fail(GFL_EINVAL, "gfl_grouped_reserve: no layer registered");
    GFL_HIP(hipSetDevice(c->device));
    Gws ws;
    // the largest layout any call up to max_picks picks can take: M <= picks tokens
    return grouped_workspace(c, nullptr, max_picks, max_picks, E, H, I, "gfl_grouped_reserve", ws);
}

int gfl_layer_info(gfl_ctx* c, int li, int* info)
{
    if (!c || !info) return fail(GFL_EINVAL, "gfl_layer_info: NULL argument");
    std::lock_guard<std::mutex> g(c->mu);
    if (li < 0 || li >= (int)c->layers.size() || !c->layers[li].dptrs)
        return fail(GFL_EINVAL, "gfl_layer_info: layer not registered");
    const Layer& L = c->layers[li];
    const int v[6] = { L.E, L.H, L.I, L.K[0], L.K[1], L.K[2] };
    for (int i = 0; i < 6; ++i) info[i] = v[i];
    return GFL_OK;
}

int gfl_grouped_plan(gfl_ctx* c, const int64_t* sel, const void* w, int w_is_half, int M, int topk, int E,
                     int* hdr, int* off, int* slot_pick, int* slot_e, int* tok_slot, float* tok_w, int* tok_npk,
                     gfl_stream stream)
{
    if (!c || !sel || !w || !hdr || !off || !slot_pick || !slot_e || !tok_slot || !tok_w || !tok_npk)
        return fail(GFL_EINVAL, "gfl_grouped_plan: NULL argument");
    if (M < 1 || topk < 1 || topk > gfl::MAX_TOPK || (int64_t)M * topk > gfl::MAX_GROUPED_PICKS)
        return fail(GFL_EINVAL, "gfl_grouped_plan: need 1 <= topk <= 16 and M*topk <= 65536");
    if (E < 1 || E > gfl::MAX_EXPERTS) return fail(GFL_EINVAL, "gfl_grouped_plan: need 1 <= E <= 1024");
    std::lock_guard<std::mutex> g(c->mu);
    GFL_HIP(hipSetDevice(c->device));
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int P = M * topk;
    Gws ws;
    if (const int rc = grouped_workspace(c, st, P, M, E, 0, 0, "gfl_grouped_plan", ws)) return rc;
    const gfl::GPlan& gp = ws.gp;
    gfl::launch_grouped_plan(sel, w, w_is_half ? 1 : 0, P, topk, E, gp, st);
    GFL_HIP(hipGetLastError());
    GFL_HIP(hipMemcpyAsync(hdr, gp.hdr, 2 * sizeof(int), hipMemcpyDeviceToDevice, st));
    GFL_HIP(hipMemcpyAsync(off, gp.off, (E + 1) * sizeof(int), hipMemcpyDeviceToDevice, st));
    GFL_HIP(hipMemcpyAsync(slot_pick, gp.slot_pick, P * sizeof(int), hipMemcpyDeviceToDevice, st));
    GFL_HIP(hipMemcpyAsync(slot_e, gp.slot_e, P * sizeof(int), hipMemcpyDeviceToDevice, st));
    GFL_HIP(hipMemcpyAsync(tok_slot, gp.tok_slot, P * sizeof(int), hipMemcpyDeviceToDevice, st));
    GFL_HIP(hipMemcpyAsync(tok_w, gp.tok_w, P * sizeof(float), hipMemcpyDeviceToDevice, st));
    GFL_HIP(hipMemcpyAsync(tok_npk, gp.tok_npk, M * sizeof(int), hipMemcpyDeviceToDevice, st));
    return GFL_OK;
}

int gfl_dequant(const void* trellis, int k, int n, int K, uint16_t* out, gfl_stream stream)
{
    if (!trellis || !out) return fail(GFL_EINVAL, "gfl_dequant: NULL argument");
    if (k < 16 || n < 16 || k % 16 || n % 16) return fail(GFL_EINVAL, "gfl_dequant: k and n must be multiples of 16");
    if (!k_ok(K)) return fail(GFL_EINVAL, "gfl_dequant: K must be 2..5");
    if (gfl::launch_dequant(static_cast<const uint8_t*>(trellis), k, n, K, out, reinterpret_cast<hipStream_t>(stream)))
        return fail(GFL_EINVAL, "gfl_dequant: unsupported K");
    GFL_HIP(hipGetLastError());
    return GFL_OK;
}

int gfl_split(const int64_t* sel, const uint16_t* w, const uint16_t* z, int bsz, int n, int H, int E, int first,
              const int32_t* slotof, const float* score, const float* pol, int64_t* ctrl, uint16_t* hx,
              int32_t* hpicks, int64_t seq, int li, int keep_ids, int64_t* sel_out, uint16_t* w_out, int64_t* dflag,
              int64_t* stats, const int32_t* rres, gfl_stream stream)
{
    if (!sel || !w || !z || !slotof || !score || !pol || !ctrl || !hx || !hpicks || !sel_out || !w_out || !dflag ||
        !stats)
        return fail(GFL_EINVAL, "gfl_split: NULL argument");
    if (bsz < 1 || n < 1 || n % bsz) return fail(GFL_EINVAL, "gfl_split: n must be a positive multiple of bsz");
    if (n > gfl::MAX_PICKS) return fail(GFL_EINVAL, "gfl_split: n <= 1024");
    if (E < 1 || E > gfl::MAX_EXPERTS || H % 8) return fail(GFL_EINVAL, "ft_split: E <= 1024");
    if ((reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(hx)) & 15)
        return fail(GFL_EINVAL, "gfl_split: z and hx must be 16-byte aligned");
    gfl::launch_split(sel, w, z, n, bsz, n / bsz, H, E, first, slotof, score, pol, ctrl, hx, hpicks, seq, li, keep_ids,
                      sel_out, w_out, dflag, stats, rres, reinterpret_cast<hipStream_t>(stream));
    GFL_HIP(hipGetLastError());
    return GFL_OK;
}

int gfl_route_split(const float* logits, int M, int E_route, int topk, int64_t* sel, uint16_t* w, const uint16_t* z,
                    int H, int E, int first, const int32_t* slotof, const float* score, const float* pol,
                    int64_t* ctrl, uint16_t* hx, int32_t* hpicks, int64_t seq, int li, int keep_ids, int64_t* sel_out,
                    uint16_t* w_out, int64_t* dflag, int64_t* stats, const int32_t* rres, gfl_stream stream)
{
    if (!logits || !sel || !w || !z || !slotof || !score || !pol || !ctrl || !hx || !hpicks || !sel_out || !w_out ||
        !dflag || !stats)
        return fail(GFL_EINVAL, "gfl_route_split: NULL argument");
    if (M < 1 || topk < 1 || topk > 64 || (int64_t)M * topk > gfl::MAX_PICKS)
        return fail(GFL_EINVAL, "gfl_route_split: need M >= 1, 1 <= topk <= 64 and M * topk <= 1024");
    if (E_route < topk || E_route > gfl::MAX_EXPERTS)
        return fail(GFL_EINVAL, "gfl_route_split: need topk <= E_route <= 1024");
    if (E < 1 || E > gfl::MAX_EXPERTS || H % 8) return fail(GFL_EINVAL, "ft_split: E <= 1024");
    if ((reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(hx)) & 15)
        return fail(GFL_EINVAL, "gfl_route_split: z and hx must be 16-byte aligned");
    if (gfl::launch_route_split(logits, M, E_route, topk, sel, w, z, H, E, first, slotof, score, pol, ctrl, hx, hpicks,
                                seq, li, keep_ids, sel_out, w_out, dflag, stats, rres,
                                reinterpret_cast<hipStream_t>(stream)))
        return fail(GFL_EINVAL, "gfl_route_split: unsupported shape");
    GFL_HIP(hipGetLastError());
    return GFL_OK;
}

int gfl_combine(void* out, int out_is_half, int n, const int64_t* dflag, const int64_t* ctrl, const float* hout,
                int64_t* stats, int64_t timeout_ns, gfl_stream stream)
{
    if (!out || !dflag || !ctrl || !hout || !stats) return fail(GFL_EINVAL, "gfl_combine: NULL argument");
    if (n < 0) return fail(GFL_EINVAL, "gfl_combine: n < 0");
    if (timeout_ns < 0) return fail(GFL_EINVAL, "gfl_combine: timeout_ns < 0");
    gfl::launch_combine(out, out_is_half ? 1 : 0, n, dflag, ctrl, hout, stats, timeout_ns,
                        reinterpret_cast<hipStream_t>(stream));
    GFL_HIP(hipGetLastError());
    return GFL_OK;
}

int gfl_grouped_rows(const int64_t* sel, const float* w, int T, int K, const uint8_t* take, int E, int32_t* experts,
                     int32_t* offsets, int32_t* row_token, float* row_weight, int* rows)
{
    if (!sel || !w || !take || !experts || !offsets || !row_token || !row_weight || !rows)
        return fail(GFL_EINVAL, "gfl_grouped_rows: NULL argument");
    if (T < 0 || K < 0 || E < 1) return fail(GFL_EINVAL, "grouped E must fit a positive int32 expert count");
    std::vector<int32_t> count((size_t)E, 0), last((size_t)E, -1), cursor((size_t)E, 0);
    for (int e = 0; e < E; ++e)
        if (take[e] > 1) return -fail(GFL_EINVAL, "grouped take entries must be zero or one");
    for (int t = 0; t < T; ++t)
        for (int k = 0; k < K; ++k)
        {
            const int64_t at = (int64_t)t * K + k, e = sel[at];
            const float wv = w[at];
            if (!std::isfinite(wv)) return -fail(GFL_EINVAL, "grouped routing weight must be finite");
            if (e < -1 || e >= E) return -fail(GFL_EINVAL, "grouped expert index out of range");
            if (e == -1)
            {
                if (wv != 0.0f) return -fail(GFL_EINVAL, "grouped masked picks require zero weight");
                continue;
            }
            if (!take[e]) continue;
            if (last[(size_t)e] == t) return -fail(GFL_EINVAL, "grouped duplicate expert for token");
            last[(size_t)e] = t;
            ++count[(size_t)e];
        }
    int nexp = 0;
    offsets[0] = 0;
    for (int e = 0; e < E; ++e)
        if (count[(size_t)e])
        {
            experts[nexp] = e;
            cursor[(size_t)e] = offsets[nexp];
            offsets[nexp + 1] = offsets[nexp] + count[(size_t)e];
            ++nexp;
        }
    for (int t = 0; t < T; ++t)
        for (int k = 0; k < K; ++k)
        {
            const int64_t at = (int64_t)t * K + k, e = sel[at];
            if (e < 0 || !take[e]) continue;
            const int32_t row = cursor[(size_t)e]++;
            row_token[row] = t;
            row_weight[row] = w[at];
        }
    *rows = offsets[nexp];
    return nexp;
}

int gfl_route(const float* logits, int M, int E, int topk, int64_t* sel, uint16_t* w, gfl_stream stream)
{
    if (M < 0) return fail(GFL_EINVAL, "gfl_route: M < 0");
    if (E < 1 || E > gfl::MAX_EXPERTS || topk < 1 || topk > E || topk > 64)
        return fail(GFL_EINVAL, "gfl_route: need 1 <= E <= 1024 and 1 <= topk <= min(E, 64)");
    if (M == 0) return GFL_OK;   // an empty batch (whose buffers may be NULL) routes nothing
    if (!logits || !sel || !w) return fail(GFL_EINVAL, "gfl_route: NULL argument");
    if (gfl::launch_route(logits, M, E, topk, sel, w, reinterpret_cast<hipStream_t>(stream)))
        return fail(GFL_EINVAL, "gfl_route: unsupported shape");
    GFL_HIP(hipGetLastError());
    return GFL_OK;
}

int gfl_synth_trellis(void* dst, size_t nbytes, uint64_t seed, gfl_stream stream)
{
    if (!dst) return fail(GFL_EINVAL, "gfl_synth_trellis: NULL destination");
    gfl::launch_synth(static_cast<uint8_t*>(dst), nbytes, seed, reinterpret_cast<hipStream_t>(stream));
    GFL_HIP(hipGetLastError());
    return GFL_OK;
}

int gfl_ingress_serve(gfl_ctx* c, int li, int bsz, int topk, int64_t* ctrl, const uint16_t* hx, const int32_t* hpicks,
                      float* hout, int mode, float act_limit, gfl_stream stream)
{
    const char* who = "gfl_ingress_serve";
    if (!c || !ctrl || !hx || !hpicks || !hout) return fail(GFL_EINVAL, std::string(who) + ": NULL argument");
    if (mode < GFL_MODE_AUTO || mode > GFL_MODE_I16)
        return fail(GFL_EINVAL, std::string(who) + ": mode must be -1 (auto), 0 (affine), 1 (exact) or 2 (i16)");
    if (const int r = check_forward(c, li, hx, c->ing_sel, c->ing_w, bsz, topk, hout, mode, act_limit, who,
                                    gfl::MAX_PICKS))
        return r;
    std::lock_guard<std::mutex> g(c->mu);
    const Layer& L = c->layers[li];
    GFL_HIP(hipSetDevice(c->device));
    if (!c->ws || L.H > c->ws_H || L.I > c->ws_I) return fail(GFL_ERUNTIME, std::string(who) + ": workspace not reserved");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    gfl::launch_ingress_take(ctrl, hpicks, li, bsz, topk, L.E, c->ing_sel, c->ing_w, c->ing_state, c->status, st);
    GFL_HIP(hipGetLastError());
    Workspace ws;
    carve_ws(c, L.H, L.I, ws);
    if (const int r = run_forward(c, L, ws, hx, c->ing_sel, c->ing_w, 0, bsz, topk, hout, mode, act_limit, st, true))
        return r;
    gfl::launch_ingress_answer(ctrl, c->ing_state, st);
    GFL_HIP(hipGetLastError());
    return GFL_OK;
}

int gfl_ctx_check(gfl_ctx* c)
{
    if (!c) return fail(GFL_EINVAL, "gfl_ctx_check: NULL context");
    std::lock_guard<std::mutex> g(c->mu);
    GFL_HIP(hipSetDevice(c->device));
    GFL_HIP(hipDeviceSynchronize());
    int w[gfl::GFL_STATUS_WORDS] = {};
    GFL_HIP(hipMemcpy(w, c->status, sizeof(w), hipMemcpyDeviceToHost));
    if (!w[gfl::GFL_STATUS_RELAY_EXPIRED] && !w[gfl::GFL_STATUS_INGRESS_REJECTED]) return GFL_OK;
    GFL_HIP(hipMemset(c->status, 0, sizeof(w)));
    GFL_HIP(hipDeviceSynchronize());
    std::string m = "gfl_ctx_check:";
    if (w[gfl::GFL_STATUS_RELAY_EXPIRED])
        m += " " + std::to_string(w[gfl::GFL_STATUS_RELAY_EXPIRED]) +
             " relay hand-off wait(s) expired (the outputs of the calls concerned are wrong);";
    if (w[gfl::GFL_STATUS_INGRESS_REJECTED])
        m += " " + std::to_string(w[gfl::GFL_STATUS_INGRESS_REJECTED]) +
             " published job(s) refused by the device worker (layer, token count, pick count, token or expert out of "
             "range; left unanswered);";
    return fail(GFL_ERUNTIME, m);
}

int gfl_ctx_set_shared(gfl_ctx* c, int shared)
{
    if (!c) return fail(GFL_EINVAL, "gfl_ctx_set_shared: NULL context");
    std::lock_guard<std::mutex> g(c->mu);
    c->shared = shared != 0;
    return GFL_OK;
}

int gfl_profile_enable(gfl_ctx* c, int enable)
{
    if (!c) return fail(GFL_EINVAL, "gfl_profile_enable: NULL context");
    std::lock_guard<std::mutex> g(c->mu);
    c->prof = enable != 0;
    return GFL_OK;
}

int gfl_profile_read(gfl_ctx* c, double* stage_ms, int64_t* launches)
{
    if (!c || !stage_ms || !launches) return fail(GFL_EINVAL, "gfl_profile_read: NULL argument");
    std::lock_guard<std::mutex> g(c->mu);
    GFL_HIP(hipSetDevice(c->device));
    for (auto& r : c->recs)
    {
        GFL_HIP(hipEventSynchronize(r.b));
        float ms = 0.f;
        GFL_HIP(hipEventElapsedTime(&ms, r.a, r.b));
        if (r.stage >= 0 && r.stage < 5)
        {
            stage_ms[r.stage] += ms;
            launches[r.stage] += 1;
        }
        c->ev_pool.push_back(r.a);
        c->ev_pool.push_back(r.b);
    }
    c->recs.clear();
    return GFL_OK;
}

int gfl_stats(gfl_ctx* c, int64_t* out, int n)
{
    if (!c || !out) return fail(GFL_EINVAL, "gfl_stats: NULL argument");
    const int64_t v[4] = { c->calls, c->picks, (int64_t)c->layers.size(), (int64_t)(c->ws_bytes + c->gws_bytes) };
    for (int i = 0; i < n && i < 4; ++i) out[i] = v[i];
    return GFL_OK;
}

}  // extern "C"
