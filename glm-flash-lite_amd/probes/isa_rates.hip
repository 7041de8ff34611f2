// Issue cost of single VALU instruction forms on gfx950 (MI355X): one workgroup of 8 waves (2 per SIMD), each wave
// running 32 independent chains of one instruction form written as inline assembly, so the measured form is exactly
// the named instruction. Prints SIMD clock cycles (s_memtime) per wave64 instruction: the slowest wave's cycles over
// (iterations x 2 waves x 32). Register-only: no memory access besides one store per thread at the end.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
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

#define CHAINS(BODY)                                                                                              \
    for (int it = 0; it < iters; ++it)                                                                            \
    {                                                                                                             \
        _Pragma("unroll") for (int i = 0; i < 32; ++i) { BODY; }                                                 \
    }

constexpr int NOPS = 30;
static const char* kNames[NOPS] = {
    "v_fmac_f32", "v_add_u32", "v_mul_lo_u32", "v_mul_u32_u24", "v_sad_u8", "v_bfe_u32", "v_alignbit_b32",
    "v_mad_u32_u16", "v_mul_lo_u16", "v_pk_fma_f16", "v_cvt_f32_f16", "v_perm_b32", "v_lshl_add_u32", "v_and_b32",
    "v_dot4_u32_u8", "v_mad_u32_u24", "v_mul_hi_u32_u24", "v_pk_mul_lo_u16", "v_xor_b32", "v_lshrrev_b32",
    "v_cvt_f32_u32", "v_fma_mix_f32", "v_mul_f32", "v_add3_u32", "v_msad_u8", "v_pk_add_u16", "v_or3_b32",
    "v_and_or_b32", "v_mul_hi_u32", "v_lshlrev_b32"};

__global__ __launch_bounds__(512) void rates(int iters, int op, unsigned* out, long long* cyc)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    unsigned u[32];
    for (int i = 0; i < 32; ++i) u[i] = lane * 7 + i * 131 + 1;
    const unsigned k = 0x83DCD12Du ^ lane, k2 = 0x3a83126fu + lane;
    __syncthreads();
    const long long t0 = clock64();
    switch (op)
    {
        case 0: CHAINS(asm volatile("v_fmac_f32 %0, %1, %2" : "+v"(u[i]) : "v"(k), "v"(k2))); break;
        case 1: CHAINS(asm volatile("v_add_u32 %0, %1, %0" : "+v"(u[i]) : "v"(k))); break;
        case 2: CHAINS(asm volatile("v_mul_lo_u32 %0, %0, %1" : "+v"(u[i]) : "v"(k))); break;
        case 3: CHAINS(asm volatile("v_mul_u32_u24 %0, %0, %1" : "+v"(u[i]) : "v"(k))); break;
        case 4: CHAINS(asm volatile("v_sad_u8 %0, %0, 0, %1" : "+v"(u[i]) : "v"(k))); break;
        case 5: CHAINS(asm volatile("v_bfe_u32 %0, %0, 5, 16" : "+v"(u[i]))); break;
        case 6: CHAINS(asm volatile("v_alignbit_b32 %0, %0, %1, 7" : "+v"(u[i]) : "v"(k))); break;
        case 7: CHAINS(asm volatile("v_mad_u32_u16 %0, %0, %1, %2" : "+v"(u[i]) : "v"(k), "v"(k2))); break;
        case 8: CHAINS(asm volatile("v_mul_lo_u16 %0, %0, %1" : "+v"(u[i]) : "v"(k))); break;
        case 9: CHAINS(asm volatile("v_pk_fma_f16 %0, %0, %1, %2" : "+v"(u[i]) : "v"(k), "v"(k2))); break;
        case 10: CHAINS(asm volatile("v_cvt_f32_f16 %0, %0" : "+v"(u[i]))); break;
        case 11: CHAINS(asm volatile("v_perm_b32 %0, %0, %1, %2" : "+v"(u[i]) : "v"(k), "v"(k2))); break;
        case 12: CHAINS(asm volatile("v_lshl_add_u32 %0, %0, 16, %1" : "+v"(u[i]) : "v"(k))); break;
        case 13: CHAINS(asm volatile("v_and_b32 %0, %0, %1" : "+v"(u[i]) : "v"(k))); break;
        case 14: CHAINS(asm volatile("v_dot4_u32_u8 %0, %0, %1, %2" : "+v"(u[i]) : "v"(k), "v"(k2))); break;
        case 15: CHAINS(asm volatile("v_mad_u32_u24 %0, %0, %1, %2" : "+v"(u[i]) : "v"(k), "v"(k2))); break;
        case 16: CHAINS(asm volatile("v_mul_hi_u32_u24 %0, %0, %1" : "+v"(u[i]) : "v"(k))); break;
        case 17: CHAINS(asm volatile("v_pk_mul_lo_u16 %0, %0, %1" : "+v"(u[i]) : "v"(k))); break;
        case 18: CHAINS(asm volatile("v_xor_b32 %0, %0, %1" : "+v"(u[i]) : "v"(k))); break;
        case 19: CHAINS(asm volatile("v_lshrrev_b32 %0, 3, %0" : "+v"(u[i]))); break;
        case 20: CHAINS(asm volatile("v_cvt_f32_u32 %0, %0" : "+v"(u[i]))); break;
        case 21: CHAINS(asm volatile("v_fma_mix_f32 %0, %0, %1, %2 op_sel_hi:[1,1,0]" : "+v"(u[i]) : "v"(k), "v"(k2))); break;
        case 22: CHAINS(asm volatile("v_mul_f32 %0, %0, %1" : "+v"(u[i]) : "v"(k))); break;
        case 23: CHAINS(asm volatile("v_add3_u32 %0, %0, %1, %2" : "+v"(u[i]) : "v"(k), "v"(k2))); break;
        case 24: CHAINS(asm volatile("v_msad_u8 %0, %0, %1, %2" : "+v"(u[i]) : "v"(k), "v"(k2))); break;
        case 25: CHAINS(asm volatile("v_pk_add_u16 %0, %0, %1" : "+v"(u[i]) : "v"(k))); break;
        case 26: CHAINS(asm volatile("v_or3_b32 %0, %0, %1, %2" : "+v"(u[i]) : "v"(k), "v"(k2))); break;
        case 27: CHAINS(asm volatile("v_and_or_b32 %0, %0, %1, %2" : "+v"(u[i]) : "v"(k), "v"(k2))); break;
        case 28: CHAINS(asm volatile("v_mul_hi_u32 %0, %0, %1" : "+v"(u[i]) : "v"(k))); break;
        case 29: CHAINS(asm volatile("v_lshlrev_b32 %0, 3, %0" : "+v"(u[i]))); break;
        default: break;
    }
    const long long t1 = clock64();
    unsigned s = 0;
    for (int i = 0; i < 32; ++i) s += u[i];
    out[threadIdx.x] = s;
    if (lane == 0) cyc[wave] = t1 - t0;
}

int main()
{
    unsigned* out;
    long long* cyc;
    HIPCHECK(hipMalloc(&out, 512 * 4));
    HIPCHECK(hipMalloc(&cyc, 8 * 8));
    const int iters = 2048;
    std::printf("| instruction | SIMD cycles per wave64 instruction |\n|---|---|\n");
    for (int op = 0; op < NOPS; ++op)
    {
        for (int rep = 0; rep < 2; ++rep)   // the first launch loads the code object
        {
            hipLaunchKernelGGL(rates, dim3(1), dim3(512), 0, 0, iters, op, out, cyc);
            HIPCHECK(hipGetLastError());
            HIPCHECK(hipDeviceSynchronize());
        }
        std::vector<long long> h(8);
        HIPCHECK(hipMemcpy(h.data(), cyc, 64, hipMemcpyDeviceToHost));
        long long mx = 0;
        for (long long x : h) mx = x > mx ? x : mx;
        std::printf("| `%s` | %.2f |\n", kNames[op], (double)mx / iters / 64.0);
    }
    return 0;
}
