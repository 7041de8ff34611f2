// Which MFMA computes the reference's EXACT chain step fmaf(x, w, acc) bit for bit, on gfx950 (MI355X), for
// fp16-valued x and w (so x * w is exact in fp32) and fp32 acc:
//   - v_mfma_f32_16x16x1_4b_f32 (K = 1: one product per output), the step of the EXACT chain GEMM;
//   - v_mfma_f32_16x16x4_4b_f16 with the weight at k = q and +0 at the other three k (one nonzero product per
//     output), which would run on the fp16 matrix path.
// One wave per trial batch: lane l passes its operands and 16 accumulators, the 16 results come back. The lane layout
// of each instruction is found first from one-hot inputs; then every output is compared with the host's fmaf on
// random magnitudes and signs, zero accumulators and accumulators that nearly cancel the product.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#define HIPCHECK(x)                                                                                               \
    do                                                                                                            \
    {                                                                                                             \
        hipError_t e_ = (x);                                                                                      \
        if (e_ != hipSuccess)                                                                                     \
        {                                                                                                         \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);                           \
            std::exit(1);                                                                                         \
        }                                                                                                         \
    } while (0)

typedef float f16v __attribute__((ext_vector_type(16)));
typedef _Float16 h4v __attribute__((ext_vector_type(4)));

// F16 = false: a, b are fp32 [trial][lane]; true: fp16 bits [trial][lane][4]
template <bool F16>
__global__ __launch_bounds__(64) void step(const void* a, const void* b, const float* c, float* d, int trials)
{
    const int l = threadIdx.x;
    for (int t = 0; t < trials; ++t)
    {
        f16v cv;
#pragma unroll
        for (int r = 0; r < 16; ++r) cv[r] = c[(t * 64 + l) * 16 + r];
        f16v dv;
        if constexpr (F16)
        {
            h4v av, bv;
            std::memcpy(&av, static_cast<const uint16_t*>(a) + (t * 64 + l) * 4, 8);
            std::memcpy(&bv, static_cast<const uint16_t*>(b) + (t * 64 + l) * 4, 8);
            dv = __builtin_amdgcn_mfma_f32_16x16x4f16(av, bv, cv, 0, 0, 0);
        }
        else
            dv = __builtin_amdgcn_mfma_f32_16x16x1f32(static_cast<const float*>(a)[t * 64 + l],
                                                      static_cast<const float*>(b)[t * 64 + l], cv, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) d[(t * 64 + l) * 16 + r] = dv[r];
    }
}

static uint16_t h16(float v)
{
    const __half x = __float2half(v);
    uint16_t u;
    std::memcpy(&u, &x, 2);
    return u;
}
static float f16(uint16_t u)
{
    __half x;
    std::memcpy(&x, &u, 2);
    return __half2float(x);
}

// a, b: per lane 1 (fp32) or 4 (fp16) operands; returns d [trials][64][16]
template <bool F16, typename T>
static std::vector<float> run(const std::vector<T>& a, const std::vector<T>& b, const std::vector<float>& c, int trials)
{
    void *da, *db;
    float *dc, *dd;
    HIPCHECK(hipMalloc(&da, a.size() * sizeof(T)));
    HIPCHECK(hipMalloc(&db, b.size() * sizeof(T)));
    HIPCHECK(hipMalloc(&dc, c.size() * 4));
    HIPCHECK(hipMalloc(&dd, c.size() * 4));
    HIPCHECK(hipMemcpy(da, a.data(), a.size() * sizeof(T), hipMemcpyHostToDevice));
    HIPCHECK(hipMemcpy(db, b.data(), b.size() * sizeof(T), hipMemcpyHostToDevice));
    HIPCHECK(hipMemcpy(dc, c.data(), c.size() * 4, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(step<F16>, dim3(1), dim3(64), 0, 0, da, db, dc, dd, trials);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipDeviceSynchronize());
    std::vector<float> d(c.size());
    HIPCHECK(hipMemcpy(d.data(), dd, c.size() * 4, hipMemcpyDeviceToHost));
    HIPCHECK(hipFree(da));
    HIPCHECK(hipFree(db));
    HIPCHECK(hipFree(dc));
    HIPCHECK(hipFree(dd));
    return d;
}

// output i = lane * 16 + register: the A lane and the B lane whose product lands there (k = 0 one-hot)
template <bool F16>
static void layout(std::vector<int>& outA, std::vector<int>& outB)
{
    outA.assign(1024, -1);
    outB.assign(1024, -1);
    const int per = F16 ? 4 : 1;
    for (int l = 0; l < 64; ++l)
        for (int side = 0; side < 2; ++side)
        {
            std::vector<float> c(1024, 0.f), d;
            if constexpr (F16)
            {
                std::vector<uint16_t> a(256, 0), b(256, 0);
                for (int i = 0; i < 64; ++i) (side ? b : a)[i * per] = h16(1.f);
                (side ? a : b)[l * per] = h16(1.f);
                d = run<true>(a, b, c, 1);
            }
            else
            {
                std::vector<float> a(64, 0.f), b(64, 0.f);
                for (int i = 0; i < 64; ++i) (side ? b : a)[i] = 1.f;
                (side ? a : b)[l] = 1.f;
                d = run<false>(a, b, c, 1);
            }
            for (int i = 0; i < 1024; ++i)
                if (d[i] != 0.f) (side ? outA : outB)[i] = l;
        }
}

int main()
{
    std::vector<int> a1, b1, a4, b4;
    layout<false>(a1, b1);
    layout<true>(a4, b4);
    int unmapped = 0, differ = 0;
    for (int i = 0; i < 1024; ++i)
    {
        unmapped += a1[i] < 0 || b1[i] < 0 || a4[i] < 0 || b4[i] < 0;
        differ += a1[i] != a4[i] || b1[i] != b4[i];
    }
    std::printf("layout: %d of 1024 outputs unmapped; %d placed differently in the two instructions\n", unmapped, differ);
    std::printf("layout: D[lane %d][reg %d] <- A lane %d, B lane %d; D[lane 17][reg 5] <- A lane %d, B lane %d\n", 0, 0,
                a1[0], b1[0], a1[17 * 16 + 5], b1[17 * 16 + 5]);

    std::mt19937 rng(12345);
    std::normal_distribution<float> nd(0.f, 1.f);
    std::uniform_int_distribution<int> ex(-30, 30);
    const int T = 4000;
    auto make_c = [&](const std::vector<float>& prod) {
        std::vector<float> c((size_t)T * 1024);
        for (size_t i = 0; i < c.size(); ++i)
        {
            float v = nd(rng) * std::ldexp(1.f, ex(rng));
            if (i % 97 == 0) v = 0.f;
            if (i % 7 == 0 && (i / 1024) % 3 == 0)   // nearly cancels the product
                v = -prod[i] * (1.f + std::ldexp(1.f, -20) * (float)((int)(i % 5) - 2));
            c[i] = v;
        }
        return c;
    };
    auto compare = [&](const char* name, const std::vector<float>& x, const std::vector<float>& w,
                       const std::vector<float>& c, const std::vector<float>& d) {
        long bad = 0;
        for (size_t i = 0; i < d.size(); ++i)
        {
            const float want = std::fmaf(x[i], w[i], c[i]);
            uint32_t wb, gb;
            std::memcpy(&wb, &want, 4);
            std::memcpy(&gb, &d[i], 4);
            if (wb != gb)
            {
                if (bad < 3)
                    std::printf("  %s: x %a w %a acc %a: fmaf %a, MFMA %a\n", name, x[i], w[i], c[i], want, d[i]);
                ++bad;
            }
        }
        std::printf("%s: %ld of %zu outputs differ from fmaf in any bit\n", name, bad, d.size());
    };
    {
        std::vector<float> a(T * 64), b(T * 64), x((size_t)T * 1024), w((size_t)T * 1024);
        for (float& v : a) v = f16(h16(nd(rng) * std::ldexp(1.f, ex(rng) / 6)));
        for (float& v : b) v = f16(h16(nd(rng) * std::ldexp(1.f, ex(rng) / 6)));
        std::vector<float> prod((size_t)T * 1024);
        for (int t = 0; t < T; ++t)
            for (int i = 0; i < 1024; ++i)
            {
                x[(size_t)t * 1024 + i] = a[t * 64 + a1[i]];
                w[(size_t)t * 1024 + i] = b[t * 64 + b1[i]];
                prod[(size_t)t * 1024 + i] = x[(size_t)t * 1024 + i] * w[(size_t)t * 1024 + i];
            }
        const std::vector<float> c = make_c(prod);
        compare("v_mfma_f32_16x16x1_4b_f32", x, w, c, run<false>(a, b, c, T));
    }
    for (int q = 0; q < 4; ++q)
    {
        std::vector<uint16_t> a(T * 256), b(T * 256, 0);
        for (uint16_t& v : a) v = h16(nd(rng) * std::ldexp(1.f, ex(rng) / 6));
        for (int i = 0; i < T * 64; ++i) b[i * 4 + q] = h16(nd(rng) * std::ldexp(1.f, ex(rng) / 6));
        std::vector<float> x((size_t)T * 1024), w((size_t)T * 1024), prod((size_t)T * 1024);
        for (int t = 0; t < T; ++t)
            for (int i = 0; i < 1024; ++i)
            {
                x[(size_t)t * 1024 + i] = f16(a[(t * 64 + a4[i]) * 4 + q]);
                w[(size_t)t * 1024 + i] = f16(b[(t * 64 + b4[i]) * 4 + q]);
                prod[(size_t)t * 1024 + i] = x[(size_t)t * 1024 + i] * w[(size_t)t * 1024 + i];
            }
        const std::vector<float> c = make_c(prod);
        char name[64];
        std::snprintf(name, sizeof name, "v_mfma_f32_16x16x4_4b_f16, product at k=%d", q);
        compare(name, x, w, c, run<true>(a, b, c, T));
    }
    return 0;
}
