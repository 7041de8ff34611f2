// PyTorch-ROCm extension over libgfl_moe.so: the torch-extension surface the reference builds from
// kernels/cpu_avx2/ft_tier_ext.cpp (tier_*, PYBIND11_MODULE at :1288-1334) and kernels/cpu_avx2/ft_tier_cu.cu
// (ft_split / ft_combine, :296-300), with the same function names, argument lists and TORCH_CHECK behaviour, so
// cpu_tier's `_H` and `_CU` handles can be this one module.
//
// With every expert resident in HBM there is no host worker pool: tier_forward runs the layer on the GPU through
// gfl_moe_forward, and the split / combine pair runs gfl_split / gfl_combine. The worker that tier_start starts is the
// device worker: while it runs, a job that ft_split publishes to the tier's ingress buffers is computed and answered
// on the split's stream right after the split (gfl_ingress_serve), as the reference's worker thread computes and
// answers every job it finds (ft_tier_ext.cpp:781-802). Work goes to the current HIP stream of the tensors' device.
// threads / cpus / swz are recorded, nothing more.
#include <torch/extension.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <string>
#include <tuple>
#include <vector>

#include "gfl_moe.h"

namespace {

hipStream_t cur_stream(const torch::Device& d) { return c10::hip::getCurrentHIPStream(d.index()).stream(); }

void check_rc(int rc)
{
    TORCH_CHECK(rc == GFL_OK, gfl_last_error());
}

struct Layer
{
    int E = 0;
    std::vector<torch::Tensor> keep;   // device copies of host-resident trellis, device scales
};

struct Tier
{
    gfl_ctx* ctx = nullptr;
    int device = 0;
    int mode = -1, H = 0, I = 0, swz = 0;
    int64_t threads = 0;
    std::vector<int64_t> cpus;
    std::vector<Layer> layers;
    std::vector<torch::Tensor> ingress;   // ctrl, hx, picks, hout (kept alive as the reference does)
    bool running = false;
    int64_t jobs = 0, experts = 0, tokens = 0, empty = 0, copied_bytes = 0;
};

Tier* T = nullptr;
float g_act_limit = 0.f;   // tier_set_act_limit may precede tier_init (ACT_LIMIT is a global in the reference)

int64_t trellis_bytes(int k, int n, int K) { return int64_t(k / 16) * (n / 16) * 32 * K; }

// Device address of a trellis the caller registered: device memory is used where it lies; host memory (the
// reference's pinned home copies) is copied once into a device buffer owned by the layer.
uint64_t device_trellis(Layer& L, int64_t addr, int64_t nbytes)
{
    hipPointerAttribute_t at{};
    const hipError_t e = hipPointerGetAttributes(&at, reinterpret_cast<const void*>(addr));
    if (e == hipSuccess && at.type == hipMemoryTypeDevice) return uint64_t(addr);
    (void)hipGetLastError();   // an unregistered (pageable) host pointer reports an error here: clear it
    auto buf = torch::empty({ nbytes }, torch::dtype(torch::kUInt8).device(torch::kCUDA, T->device));
    const hipError_t c = hipMemcpy(buf.data_ptr(), reinterpret_cast<const void*>(addr), size_t(nbytes),
                                   hipMemcpyHostToDevice);
    TORCH_CHECK(c == hipSuccess, "tier_add_layer: trellis copy to the device failed: ", hipGetErrorString(c));
    L.keep.push_back(buf);
    T->copied_bytes += nbytes;
    return uint64_t(reinterpret_cast<uintptr_t>(buf.data_ptr()));
}

}  // namespace

// ---- tier_* (ft_tier_ext.cpp) -------------------------------------------------------------------------------

void tier_init(int64_t threads, std::vector<int64_t> cpus, torch::Tensor ctrl, torch::Tensor hx, torch::Tensor picks,
               torch::Tensor hout, int64_t mode, int64_t H, int64_t I, int64_t nlayers, int64_t swz)
{
    TORCH_CHECK(T == nullptr, "tier already initialised");
    TORCH_CHECK(mode >= -1 && mode <= 2, "tier_init: mode must be -1, 0, 1 or 2");
    TORCH_CHECK(H >= 256 && I >= 256 && H % 256 == 0 && I % 256 == 0, "tier_init: H and I must be multiples of 256");
    TORCH_CHECK(nlayers >= 0 && nlayers <= 4096, "tier_init: layer count out of range");
    int dev = 0;
    TORCH_CHECK(hipGetDevice(&dev) == hipSuccess, "tier_init: no GPU (the expert path runs on the device)");
    gfl_ctx* ctx = nullptr;
    check_rc(gfl_ctx_create(dev, &ctx));
    T = new Tier();
    T->ctx = ctx;
    T->device = dev;
    T->mode = int(mode); T->H = int(H); T->I = int(I); T->swz = int(swz);
    T->threads = threads; T->cpus = cpus;
    T->layers.resize(size_t(nlayers));
    T->ingress = { ctrl, hx, picks, hout };
}

// Release the singleton (the reference process never does; tests and re-initialisation do).
void tier_shutdown()
{
    if (!T) return;
    hipDeviceSynchronize();
    gfl_ctx_destroy(T->ctx);
    delete T;
    T = nullptr;
}

// ptrs: int64 [E, 3] addresses of the gate/up/down trellis (native [k/16][n/16] tile layout), device memory or host
// memory (copied to the device here); scales fp16 [E, .] on the CPU or on the device. bits extends the reference's
// fixed K=3 to mixed-bitrate layers (2..5 per matrix).
void tier_add_layer(int64_t li, torch::Tensor ptrs, torch::Tensor suh_g, torch::Tensor svh_g, torch::Tensor suh_u,
                    torch::Tensor svh_u, torch::Tensor suh_d, torch::Tensor svh_d, std::vector<int64_t> bits)
{
    TORCH_CHECK(T, "init first");
    TORCH_CHECK(li >= 0 && li < int64_t(T->layers.size()), "tier_add_layer: layer index out of range");
    TORCH_CHECK(ptrs.scalar_type() == at::kLong && ptrs.dim() == 2 && ptrs.size(1) == 3, "ptrs: int64 [E, 3]");
    TORCH_CHECK(bits.size() == 3, "tier_add_layer: bits = (k_gate, k_up, k_down)");
    const int E = int(ptrs.size(0)), H = T->H, I = T->I;
    for (const auto& t : { suh_g, svh_g, suh_u, svh_u, suh_d, svh_d })
        TORCH_CHECK(t.scalar_type() == at::kHalf && t.is_contiguous() && t.dim() == 2 && t.size(0) == E,
                    "scales: CPU fp16 contiguous [E, .]");
    TORCH_CHECK(suh_g.size(1) == H && svh_g.size(1) == I && suh_u.size(1) == H && svh_u.size(1) == I &&
                    suh_d.size(1) == I && svh_d.size(1) == H,
                "scale shapes");
    const c10::DeviceGuard g(torch::Device(torch::kCUDA, T->device));
    Layer L;
    std::vector<torch::Tensor> sc;
    for (const auto& t : { suh_g, svh_g, suh_u, svh_u, suh_d, svh_d })
    {
        sc.push_back(t.to(torch::Device(torch::kCUDA, T->device)).contiguous());
        L.keep.push_back(sc.back());
    }
    const auto p = ptrs.cpu().contiguous();
    const int64_t* pa = p.data_ptr<int64_t>();
    const int dims[3][2] = { { H, I }, { H, I }, { I, H } };
    std::vector<uint64_t> table(size_t(E) * 9);
    for (int e = 0; e < E; ++e)
    {
        for (int m = 0; m < 3; ++m)
            table[size_t(e) * 9 + m] =
                device_trellis(L, pa[e * 3 + m], trellis_bytes(dims[m][0], dims[m][1], int(bits[m])));
        for (int s = 0; s < 6; ++s)
            table[size_t(e) * 9 + 3 + s] =
                uint64_t(reinterpret_cast<uintptr_t>(sc[s].data_ptr())) + uint64_t(e) * sc[s].size(1) * 2;
    }
    check_rc(gfl_register_layer(T->ctx, int(li), E, H, I, int(bits[0]), int(bits[1]), int(bits[2]), table.data()));
    L.keep.push_back(ptrs);
    L.E = E;
    T->layers[size_t(li)] = std::move(L);
}

// Starts the device worker (the reference pins a worker thread to cpu0, ft_tier_ext.cpp:781-802; here the jobs are
// served on the device, so cpu0 is recorded only).
void tier_start(int64_t cpu0)
{
    TORCH_CHECK(T && !T->running, "init first / already running");
    (void)cpu0;
    T->running = true;
}

void tier_stop()
{
    if (!T) return;
    T->running = false;
}

// Every mode number of the reference is accepted, and every one computes EXACT, bit-identical to the reference's
// EXACT mode at every size up to 65,536 picks (as gfl_moe_forward does for them): the reference CPU engine's speed
// modes (-1 auto, 0 AFFINE, 2 I16, ft_tier_ext.cpp:396) trade accuracy for CPU time, and EXACT lies closer to the fp64
// expert than either. The MFMA grouped path (gfl_grouped_forward) is not reached from here.
torch::Tensor tier_forward(int64_t li, torch::Tensor x, torch::Tensor sel, torch::Tensor w, int64_t mode)
{
    TORCH_CHECK(T && !T->running, "tier_forward: worker running");
    TORCH_CHECK(li >= 0 && li < int64_t(T->layers.size()) && T->layers[size_t(li)].E > 0,
                "tier_forward: layer not registered");
    TORCH_CHECK(mode >= -1 && mode <= 2, "tier_forward: mode must be -1, 0, 1 or 2");
    TORCH_CHECK(x.scalar_type() == at::kFloat && x.dim() == 2 && x.size(1) == T->H, "x: float32 [m, H]");
    TORCH_CHECK((sel.scalar_type() == at::kInt || sel.scalar_type() == at::kLong) && sel.dim() == 2 &&
                    sel.size(0) == x.size(0),
                "sel: int32 [m, k]");
    TORCH_CHECK(w.scalar_type() == at::kFloat && w.sizes() == sel.sizes(), "w: float32 [m, k]");
    const int64_t m = x.size(0), k = sel.size(1);
    // m = 0 gives an empty [0, H] result and k = 0 zeros, as the reference's tier_forward does (ft_tier_ext.cpp:893-903)
    TORCH_CHECK(k <= 16 && m * k <= 65536, "tier_forward: k <= 16 and m * k <= 65536 picks");
    const torch::Device dev(torch::kCUDA, T->device);
    const c10::DeviceGuard g(dev);
    auto xd = x.to(dev);
    auto x16 = xd.to(torch::kHalf).contiguous();
    TORCH_CHECK(torch::equal(x16.to(torch::kFloat), xd),
                "tier_forward: x must be fp16-valued (the expert input is fp16)");
    const int E = T->layers[size_t(li)].E;
    TORCH_CHECK(sel.lt(E).all().item<bool>(), "tier_forward: expert id out of range");
    auto seld = sel.to(dev).to(torch::kLong);
    seld = torch::where(seld.lt(0), torch::full_like(seld, -1), seld).contiguous();
    auto wd = w.to(dev).contiguous();
    auto out = torch::empty({ m, int64_t(T->H) }, torch::dtype(torch::kFloat).device(dev));
    const hipStream_t st = cur_stream(dev);
    check_rc(gfl_moe_forward(T->ctx, int(li), static_cast<const uint16_t*>(x16.data_ptr()), seld.data_ptr<int64_t>(),
                             wd.data_ptr(), 0, int(m), int(k), out.data_ptr<float>(), int(mode), g_act_limit, st));
    const int64_t valid = sel.ge(0).sum().item<int64_t>();
    T->jobs += 1;
    T->experts += valid;
    T->tokens += m;
    T->empty += valid == 0;
    return x.is_cuda() ? out : out.cpu();
}

// [jobs, experts, tokens, empty, busy_ns, swz_bytes, phase ns x5, prep ns] (ft_tier_ext.cpp:906-914). Counts are of
// tier_forward calls (there is no host worker); swz_bytes holds the bytes of host trellis copied to the device at
// registration; the host phase times have no counterpart.
std::vector<int64_t> tier_stats()
{
    if (!T) return {};
    return { T->jobs, T->experts, T->tokens, T->empty, 0, T->copied_bytes, 0, 0, 0, 0, 0, 0 };
}

void tier_set_act_limit(double limit)
{
    g_act_limit = float(limit);
}

// [E6] CPU-job schedule switches (ft_tier_ext.cpp:806-812): recorded and echoed; no CPU job schedule exists here.
std::vector<int64_t> tier_set_e6(int64_t fuse, int64_t fuse_maxn, int64_t lean)
{
    static int64_t v[3] = { 0, 1, 0 };
    if (fuse >= 0) v[0] = fuse;
    if (fuse_maxn >= 0) v[1] = fuse_maxn;
    if (lean >= 0) v[2] = lean;
    return { v[0], v[1], v[2] };
}

// Per-bucket host job histogram (ft_tier_ext.cpp:659-666): 17 buckets x (jobs, busy, local, wait), all zero (no host
// jobs run).
std::vector<int64_t> tier_job_hist()
{
    if (!T) return {};
    return std::vector<int64_t>(17 * 4, 0);
}

// ft_tier_ext.cpp:1047-1097 -> (experts int32, offsets int32 [n+1], row_token int32, row_weight float32) on the CPU
std::vector<torch::Tensor> tier_lut_build_grouped_rows(torch::Tensor sel, torch::Tensor w, torch::Tensor take,
                                                       int64_t E)
{
    TORCH_CHECK(E >= 1 && E < 2147483647LL, "grouped E must fit a positive int32 expert count");
    TORCH_CHECK(sel.device().is_cpu() && sel.scalar_type() == at::kLong && sel.is_contiguous() && sel.dim() == 2,
                "grouped sel must be contiguous CPU int64 [T,K] with int32-sized rows");
    TORCH_CHECK(w.device().is_cpu() && (w.scalar_type() == at::kHalf || w.scalar_type() == at::kFloat) &&
                    w.is_contiguous() && w.sizes() == sel.sizes(),
                "grouped weights must match sel as contiguous CPU fp16 or float32");
    TORCH_CHECK(take.device().is_cpu() && take.scalar_type() == at::kByte && take.is_contiguous() && take.dim() == 1 &&
                    take.numel() == E,
                "grouped take must be contiguous CPU uint8 [E]");
    const int Tn = int(sel.size(0)), K = int(sel.size(1));
    auto wf = w.to(torch::kFloat).contiguous();
    auto ex = torch::zeros({ E }, torch::kInt);
    auto off = torch::zeros({ E + 1 }, torch::kInt);
    auto rt = torch::zeros({ std::max<int64_t>(1, int64_t(Tn) * K) }, torch::kInt);
    auto rw = torch::zeros({ std::max<int64_t>(1, int64_t(Tn) * K) }, torch::kFloat);
    int rows = 0;
    const int n = gfl_grouped_rows(sel.data_ptr<int64_t>(), wf.data_ptr<float>(), Tn, K, take.data_ptr<uint8_t>(),
                                   int(E), ex.data_ptr<int32_t>(), off.data_ptr<int32_t>(), rt.data_ptr<int32_t>(),
                                   rw.data_ptr<float>(), &rows);
    TORCH_CHECK(n >= 0, gfl_last_error());
    return { ex.narrow(0, 0, n).clone(), off.narrow(0, 0, n + 1).clone(), rt.narrow(0, 0, rows).clone(),
             rw.narrow(0, 0, rows).clone() };
}

// ---- ft_split / ft_combine (ft_tier_cu.cu) ---------------------------------------------------------------------

void ft_split(torch::Tensor sel, torch::Tensor w, torch::Tensor z, int64_t E, int64_t first, torch::Tensor slotof,
              torch::Tensor score, torch::Tensor pol, int64_t ctrl, int64_t hx, int64_t hpicks, int64_t seq, int64_t li,
              int64_t keep_ids, torch::Tensor sel_out, torch::Tensor w_out, torch::Tensor dflag, torch::Tensor stats,
              torch::Tensor rres)
{
    TORCH_CHECK(pol.numel() >= 20, "ft_split: policy needs 20 entries");
    TORCH_CHECK(rres.numel() == 0 || (rres.scalar_type() == at::kInt && rres.numel() >= E),
                "ft_split: rres int32 [E] or empty");
    TORCH_CHECK(sel.scalar_type() == at::kLong && w.scalar_type() == at::kHalf && z.scalar_type() == at::kHalf &&
                    z.is_contiguous(),
                "dtypes");
    TORCH_CHECK(z.dim() == 2, "ft_split: z [bsz, H]");
    const int bsz = int(z.size(0)), H = int(z.size(1)), n = int(sel.numel());
    TORCH_CHECK(E <= 1024 && H % 8 == 0, "ft_split: E <= 1024");
    TORCH_CHECK(bsz >= 1 && n % bsz == 0 && n <= 1024, "ft_split: sel holds bsz * topk <= 1024 picks");
    for (const auto& t : { sel, w, slotof, score, pol, sel_out, w_out, dflag, stats })
        TORCH_CHECK(t.is_cuda() && t.device() == sel.device() && t.is_contiguous(),
                    "ft_split: buffers on one device, contiguous");
    TORCH_CHECK(slotof.scalar_type() == at::kInt && slotof.numel() >= E && score.scalar_type() == at::kFloat &&
                    score.numel() >= E && pol.scalar_type() == at::kFloat && sel_out.scalar_type() == at::kLong &&
                    sel_out.numel() >= n && w_out.scalar_type() == at::kHalf && w_out.numel() >= n &&
                    dflag.scalar_type() == at::kLong && stats.scalar_type() == at::kLong && stats.numel() >= 8,
                "ft_split: buffer dtype/capacity mismatch");
    const c10::DeviceGuard g(sel.device());
    check_rc(gfl_split(sel.data_ptr<int64_t>(), static_cast<const uint16_t*>(w.data_ptr()),
                       static_cast<const uint16_t*>(z.data_ptr()), bsz, n, H, int(E), int(first),
                       slotof.data_ptr<int32_t>(), score.data_ptr<float>(), pol.data_ptr<float>(),
                       reinterpret_cast<int64_t*>(ctrl), reinterpret_cast<uint16_t*>(hx),
                       reinterpret_cast<int32_t*>(hpicks), seq, int(li), int(keep_ids), sel_out.data_ptr<int64_t>(),
                       static_cast<uint16_t*>(w_out.data_ptr()), dflag.data_ptr<int64_t>(), stats.data_ptr<int64_t>(),
                       rres.numel() ? rres.data_ptr<int32_t>() : nullptr, cur_stream(sel.device())));
    // the device worker serves the tier's own ingress buffers while it runs (a split on other buffers is left to
    // whoever consumes them)
    if (T && T->running && ctrl == reinterpret_cast<int64_t>(T->ingress[0].data_ptr()))
    {
        const int li_ = int(li);
        TORCH_CHECK(li_ >= 0 && li_ < int(T->layers.size()) && T->layers[size_t(li_)].E > 0,
                    "ft_split: the tier's worker has no layer ", li_);
        check_rc(gfl_ingress_serve(T->ctx, li_, bsz, n / bsz, reinterpret_cast<int64_t*>(ctrl),
                                   reinterpret_cast<const uint16_t*>(hx), reinterpret_cast<const int32_t*>(hpicks),
                                   static_cast<float*>(T->ingress[3].data_ptr()), T->mode, g_act_limit,
                                   cur_stream(sel.device())));
    }
}

void ft_combine(torch::Tensor out, torch::Tensor dflag, int64_t ctrl, int64_t hout, torch::Tensor stats,
                int64_t timeout_ns)
{
    TORCH_CHECK(out.is_contiguous() && (out.scalar_type() == at::kFloat || out.scalar_type() == at::kHalf),
                "out fp32/fp16 contiguous");
    TORCH_CHECK(dflag.scalar_type() == at::kLong && stats.scalar_type() == at::kLong && stats.numel() >= 8,
                "ft_combine: dtypes");
    TORCH_CHECK(out.is_cuda() && dflag.device() == out.device() && stats.device() == out.device(),
                "ft_combine: buffers on one device");
    const c10::DeviceGuard g(out.device());
    check_rc(gfl_combine(out.data_ptr(), out.scalar_type() == at::kHalf ? 1 : 0, int(out.numel()),
                         dflag.data_ptr<int64_t>(), reinterpret_cast<const int64_t*>(ctrl),
                         reinterpret_cast<const float*>(hout), stats.data_ptr<int64_t>(), timeout_ns,
                         cur_stream(out.device())));
}

// No counterpart in the reference: (initialised, running, act_limit, layers registered) for the serve-layer stats.
std::tuple<bool, bool, double, int64_t> tier_state()
{
    if (!T) return { false, false, double(g_act_limit), 0 };
    int64_t n = 0;
    for (const auto& L : T->layers) n += L.E > 0;
    return { true, T->running, double(g_act_limit), n };
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m)
{
    m.def("tier_init", &tier_init);
    m.def("tier_add_layer", &tier_add_layer, pybind11::arg("li"), pybind11::arg("ptrs"), pybind11::arg("suh_g"),
          pybind11::arg("svh_g"), pybind11::arg("suh_u"), pybind11::arg("svh_u"), pybind11::arg("suh_d"),
          pybind11::arg("svh_d"), pybind11::arg("bits") = std::vector<int64_t>{ 3, 3, 3 });
    m.def("tier_start", &tier_start);
    m.def("tier_stop", &tier_stop);
    m.def("tier_forward", &tier_forward);
    m.def("tier_stats", &tier_stats);
    m.def("tier_set_act_limit", &tier_set_act_limit);
    m.def("tier_set_e6", &tier_set_e6);
    m.def("tier_job_hist", &tier_job_hist);
    m.def("tier_lut_build_grouped_rows", &tier_lut_build_grouped_rows, pybind11::arg("sel"), pybind11::arg("w"),
          pybind11::arg("take"), pybind11::arg("E"));
    m.def("tier_shutdown", &tier_shutdown);
    m.def("tier_state", &tier_state);
    m.def("ft_split", &ft_split);
    m.def("ft_combine", &ft_combine);
}
