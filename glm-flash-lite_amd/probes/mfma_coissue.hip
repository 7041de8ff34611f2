// Whether VALU instructions issue while the matrix cores run, on gfx950 (MI355X). One workgroup; wave w runs on SIMD
// w % 4 and takes the role given by digit w of the case string:
//   0: 4 independent accumulations of v_mfma_f32_16x16x1_4b_f32 (the EXACT chain GEMM's step) per iteration
//   1: 32 independent v_fmac_f32 per iteration (VALU)
//   2: 4 independent v_mfma_f32_16x16x16_f16 per iteration
//   3: 4 independent v_mfma_f32_16x16x4_4b_f16 per iteration
// Printed: each wave's s_memtime cycles per iteration. A SIMD whose MFMA waves keep their alone-rate while its VALU
// wave also keeps its alone-rate co-issues; a VALU wave slowed by the MFMA waves' busy cycles does not. Register-only.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <cstring>
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
typedef float f4v __attribute__((ext_vector_type(4)));
typedef _Float16 h4v __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(1024) void roles_kernel(int iters, const int* roles, float* out, long long* cyc)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int role = roles[wave];
    float s = 0.f;
    __syncthreads();
    const long long t0 = clock64();
    if (role == 0)
    {
        f16v acc[4];
        for (int c = 0; c < 4; ++c)
            for (int r = 0; r < 16; ++r) acc[c][r] = 0.f;
        const float a = 1.0f + lane * 1e-3f, b = 0.5f + wave * 1e-3f;
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, acc[c], 0, 0, 0);
        for (int c = 0; c < 4; ++c)
            for (int r = 0; r < 16; ++r) s += acc[c][r];
    }
    else if (role == 1)
    {
        float v[32];
        for (int i = 0; i < 32; ++i) v[i] = lane + i;
        const float y = 0.999f + lane * 1e-6f;
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int i = 0; i < 32; ++i) v[i] = __builtin_fmaf(v[i], y, 1e-3f);
        for (int i = 0; i < 32; ++i) s += v[i];
    }
    else if (role == 2)
    {
        f4v acc[4];
        for (int c = 0; c < 4; ++c) acc[c] = f4v{0.f, 0.f, 0.f, 0.f};
        const h4v ha = {(_Float16)1.0f, (_Float16)0.5f, (_Float16)(lane * 1e-3f), (_Float16)0.25f};
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(ha, ha, acc[c], 0, 0, 0);
        for (int c = 0; c < 4; ++c) s += acc[c][0] + acc[c][3];
    }
    else if (role == 3)
    {
        f16v acc[4];
        for (int c = 0; c < 4; ++c)
            for (int r = 0; r < 16; ++r) acc[c][r] = 0.f;
        const h4v ha = {(_Float16)1.0f, (_Float16)0.0f, (_Float16)(lane * 1e-3f), (_Float16)0.0f};
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f16(ha, ha, acc[c], 0, 0, 0);
        for (int c = 0; c < 4; ++c)
            for (int r = 0; r < 16; ++r) s += acc[c][r];
    }
    const long long t1 = clock64();
    out[threadIdx.x] = s;
    if (lane == 0) cyc[wave] = t1 - t0;
}

int main()
{
    float* out;
    long long* cyc;
    int* roles;
    HIPCHECK(hipMalloc(&out, 1024 * 4));
    HIPCHECK(hipMalloc(&cyc, 16 * 8));
    HIPCHECK(hipMalloc(&roles, 16 * 4));
    const int iters = 4096;
    const char* cases[] = {"0000", "00000000", "1111", "11111111", "2222", "3333", "00001111", "000000001111",
                           "0000000011111111", "22221111", "222222221111", "33331111", "333333331111"};
    std::printf("| waves (role per wave) | cycles per iteration, per wave |\n|---|---|\n");
    for (const char* c : cases)
    {
        const int nw = (int)std::strlen(c);
        std::vector<int> r(nw);
        for (int i = 0; i < nw; ++i) r[i] = c[i] - '0';
        HIPCHECK(hipMemcpy(roles, r.data(), nw * 4, hipMemcpyHostToDevice));
        for (int rep = 0; rep < 2; ++rep)
        {
            hipLaunchKernelGGL(roles_kernel, dim3(1), dim3(nw * 64), 0, 0, iters, roles, out, cyc);
            HIPCHECK(hipGetLastError());
            HIPCHECK(hipDeviceSynchronize());
        }
        std::vector<long long> h(nw);
        HIPCHECK(hipMemcpy(h.data(), cyc, nw * 8, hipMemcpyDeviceToHost));
        std::printf("| %s |", c);
        for (int i = 0; i < nw; ++i) std::printf(" %.0f", (double)h[i] / iters);
        std::printf(" |\n");
    }
    return 0;
}
