// The trellis decode step of the relay GEMV loop with the codebook computed or looked up, on gfx950 (MI355X). Each
// wave runs the inner loop on LDS-resident data: per group of 8 tiles (K = 3) it rewrites its 768-byte slot from a
// register LCG (as the relay kernel writes each group from registers), decodes the 8 tiles (two LDS words per lane
// per tile), transposes each by one MFMA and runs the 32 chain FMAs against fp32 inputs read from LDS ([tile][j][q]).
//   V = 0: the library's decode (decode4: v_mul_lo_u32 MUL1 hash, v_sad_u8 byte sums, v_pk_fma_f16);
//   V = 1: a 65,536-entry fp16 LDS table (128 KB) indexed by the 16-bit state, for all 4 weights of a lane;
//   V = 2: the table for weights 0 and 1 only, the computed codebook for 2 and 3;
//   V = 3: a per-lane recurrence of the hash products: p_{t+1} = (p_t << K) + T[top K bits of s_t, next K bits]
//          mod 2^32 with a 64-entry LDS table T, one v_mul_lo_u32 per 4 states instead of 4.
// Every variant's outputs are compared with V = 0's bit for bit. Times: 3 launches of 256 workgroups (one per CU) at
// 4..16 waves per workgroup; "pmc" runs one launch of each variant at 16 waves, for counter passes. All LDS
// addresses are masked into their arrays; loops have fixed trip counts; one global store per thread.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include <cstring>
#include <vector>
#include "../csrc/gfl_device.hpp"
using namespace gfl;

constexpr int K = 3, TB = 32 * K, GB = 8 * TB;   // 96-byte tiles, 768-byte groups
constexpr int XIN = 5120;                         // inputs per slot (fp32): 20 KB
constexpr int TAB_BYTES = 131072;
constexpr int REC_OFF = 0;   // the recurrence table (V = 3 only) in the space of the 128 KB table, which V = 3 leaves unused

// codebook4 after the hash multiply: products -> fp16 weights
__device__ inline half4 codebook_p(uint32_t p0, uint32_t p1, uint32_t p2, uint32_t p3)
{
    uint32_t s01 = __builtin_amdgcn_sad_u8(p0, 0u, 0x64006400u);
    uint32_t s23 = __builtin_amdgcn_sad_u8(p2, 0u, 0x64006400u);
    asm("v_sad_hi_u8 %0, %1, 0, %0" : "+v"(s01) : "v"(p1));
    asm("v_sad_hi_u8 %0, %1, 0, %0" : "+v"(s23) : "v"(p3));
    half2v a, b;
    __builtin_memcpy(&a, &s01, 4);
    __builtin_memcpy(&b, &s23, 4);
    _Float16 ki, kb;
    const uint16_t kib = KINV_BITS, kbb = KBIAS_BITS;
    __builtin_memcpy(&ki, &kib, 2);
    __builtin_memcpy(&kb, &kbb, 2);
    const half2v kinv2 = { ki, ki }, kbias2 = { kb, kb };
    const half2v w01 = __builtin_elementwise_fma(a, kinv2, kbias2);
    const half2v w23 = __builtin_elementwise_fma(b, kinv2, kbias2);
    half4 r = { w01[0], w01[1], w23[0], w23[1] };
    return r;
}

// the four states of decode4 (s_i = bits [(3 - i) K, (3 - i) K + 16) of the window) by the recurrence
__device__ inline half4 dec_rec(uint32_t hi, uint32_t lo, uint32_t sh, const uint32_t* T)
{
    const uint32_t R = __builtin_amdgcn_alignbit(hi, lo, sh);
    uint32_t p[4];
    p[0] = __builtin_amdgcn_ubfe(R, 3 * K, 16) * MUL1;
#pragma unroll
    for (int i = 0; i < 3; ++i)
    {
        const uint32_t y = R >> ((2 - i) * K);   // next K bits at 0..K-1, the top K bits of s_i at 16..16+K-1
        const uint32_t idx = (y & 7u) | ((y >> 13) & 0x38u);
        p[i + 1] = (p[i] << K) + T[idx];
    }
    return codebook_p(p[0], p[1], p[2], p[3]);
}

template <int V>
__device__ __forceinline__ half4 dec_tab(uint32_t hi, uint32_t lo, uint32_t sh, const uint8_t* tb)
{
    const uint32_t R = __builtin_amdgcn_alignbit(hi, lo, sh);
    if constexpr (V == 1)
    {
        const uint32_t a0 = (R >> (3 * K - 1)) & 0x1FFFEu, a1 = (R >> (2 * K - 1)) & 0x1FFFEu;
        const uint32_t a2 = (R >> (K - 1)) & 0x1FFFEu, a3 = (R << 1) & 0x1FFFEu;
        half4 r;
        r[0] = *reinterpret_cast<const _Float16*>(tb + a0);
        r[1] = *reinterpret_cast<const _Float16*>(tb + a1);
        r[2] = *reinterpret_cast<const _Float16*>(tb + a2);
        r[3] = *reinterpret_cast<const _Float16*>(tb + a3);
        return r;
    }
    else
    {
        const uint32_t a0 = (R >> (3 * K - 1)) & 0x1FFFEu, a1 = (R >> (2 * K - 1)) & 0x1FFFEu;
        const half4 c = codebook4(0u, 0u, __builtin_amdgcn_ubfe(R, K, 16), __builtin_amdgcn_ubfe(R, 0, 16));
        half4 r;
        r[0] = *reinterpret_cast<const _Float16*>(tb + a0);
        r[1] = *reinterpret_cast<const _Float16*>(tb + a1);
        r[2] = c[2];
        r[3] = c[3];
        return r;
    }
}

template <int V>
__global__ __launch_bounds__(1024) void probe(float* out, int ngroups, uint32_t seed, int fill)
{
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t* tab = lds;                                   // [65536] fp16
    float* xin = reinterpret_cast<float*>(lds + TAB_BYTES);   // [XIN]
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    uint8_t* slot = lds + TAB_BYTES + XIN * 4 + wave * GB;
    // inputs: fp16-valued fp32
    for (int i = threadIdx.x; i < XIN; i += blockDim.x)
        xin[i] = (float)(_Float16)((float)((i * 2654435761u) >> 20) / 4096.0f - 0.5f);
    if (V != 0 || fill)
        for (int i = threadIdx.x; i < 16384; i += blockDim.x)
        {
            const half4 c = codebook4(4 * i, 4 * i + 1, 4 * i + 2, 4 * i + 3);
            *reinterpret_cast<half4*>(tab + 8 * i) = c;
        }
    uint32_t* rtab = reinterpret_cast<uint32_t*>(lds + REC_OFF);
    if (V == 3 && threadIdx.x < 64)
    {
        const uint32_t top = threadIdx.x >> 3, nw = threadIdx.x & 7;   // T[top, new] = new C - (top C) << 16
        rtab[threadIdx.x] = nw * MUL1 - ((top * MUL1) << 16);
    }
    __syncthreads();
    const LaneDec d = lane_dec(lane, K);
    const int j = lane >> 4, n = lane & 15;
    half4 Pm;
#pragma unroll
    for (int r = 0; r < 4; ++r) Pm[r] = (_Float16)((j == (n & 3) && r == (n >> 2)) ? 1.0f : 0.0f);
    const float4v zero = { 0.f, 0.f, 0.f, 0.f };
    uint32_t s0 = seed ^ (blockIdx.x * 7919u + threadIdx.x * 104729u), s1 = s0 * 747796405u + 2891336453u,
             s2 = s1 * 747796405u + 2891336453u;
    float acc = 0.f;
    for (int g = 0; g < ngroups; ++g)
    {
        // rewrite the slot: 768 bytes = 3 dwords per lane
        s0 = s0 * 1664525u + 1013904223u; s1 = s1 * 1664525u + 1013904223u; s2 = s2 * 1664525u + 1013904223u;
        uint32_t* sw = reinterpret_cast<uint32_t*>(slot);
        sw[lane] = s0; sw[64 + lane] = s1; sw[128 + lane] = s2;
        float4v cw[8], xf[8];
#pragma unroll
        for (int rr = 0; rr < 8; ++rr)
        {
            const uint8_t* tp = slot + rr * TB;
            const uint32_t hi = *reinterpret_cast<const uint32_t*>(tp + d.o0);
            const uint32_t lo = *reinterpret_cast<const uint32_t*>(tp + d.o1);
            half4 wv;
            if constexpr (V == 0) wv = decode4<K>(hi, lo, d.sh);
            else if constexpr (V == 3) wv = dec_rec(hi, lo, d.sh, rtab);
            else wv = dec_tab<V>(hi, lo, d.sh, tab);
            cw[rr] = __builtin_amdgcn_mfma_f32_16x16x16f16(Pm, wv, zero, 0, 0, 0);
        }
        const int gi = g % (XIN / 128);
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) xf[rr] = *reinterpret_cast<const float4v*>(xin + (gi * 8 + rr) * 16 + j * 4);
#pragma unroll
        for (int rr = 0; rr < 8; ++rr)
        {
            acc = __builtin_fmaf(cw[rr][0], xf[rr][0], acc);
            acc = __builtin_fmaf(cw[rr][1], xf[rr][1], acc);
            acc = __builtin_fmaf(cw[rr][2], xf[rr][2], acc);
            acc = __builtin_fmaf(cw[rr][3], xf[rr][3], acc);
        }
    }
    out[blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

template <int V>
double run(int waves, int ngroups, int nblk, std::vector<float>& host, int fill)
{
    const size_t lds = TAB_BYTES + XIN * 4 + waves * GB;
    hipFuncSetAttribute((const void*)probe<V>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    float* d = nullptr;
    hipMalloc(&d, (size_t)nblk * waves * 64 * 4);
    hipEvent_t a, b;
    hipEventCreate(&a); hipEventCreate(&b);
    hipLaunchKernelGGL(probe<V>, dim3(nblk), dim3(waves * 64), lds, 0, d, ngroups, 12345u, fill);
    hipEventRecord(a);
    for (int r = 0; r < 3; ++r)
        hipLaunchKernelGGL(probe<V>, dim3(nblk), dim3(waves * 64), lds, 0, d, ngroups, 12345u, fill);
    hipEventRecord(b);
    hipEventSynchronize(b);
    float ms = 0;
    hipEventElapsedTime(&ms, a, b);
    host.resize((size_t)nblk * waves * 64);
    hipMemcpy(host.data(), d, host.size() * 4, hipMemcpyDeviceToHost);
    hipFree(d);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) { printf("HIP error %s\n", hipGetErrorString(e)); exit(1); }
    return ms / 3.0;
}

int main(int argc, char** argv)
{
    const int nblk = 256;
    if (argc > 1 && !strcmp(argv[1], "pmc"))
    {
        // one dispatch per variant at 16 waves per workgroup, for counter runs (dispatches 1-4: computed, 5-8: table,
        // 9-12: half-table, 13-16: recurrence; each run() is a warm-up launch and 3 timed ones)
        std::vector<float> h;
        const double t0 = run<0>(16, 200, nblk, h, 0), t1 = run<1>(16, 200, nblk, h, 1),
                     t2 = run<2>(16, 200, nblk, h, 1), t3 = run<3>(16, 200, nblk, h, 0);
        printf("pmc pass: computed %.1f us, table %.1f us, half-table %.1f us, recurrence %.1f us (tiles per dispatch "
               "%d)\n", t0 * 1e3, t1 * 1e3, t2 * 1e3, t3 * 1e3, nblk * 16 * 200 * 8);
        return 0;
    }
    printf("per CU: one workgroup (128 KB table + 20 KB inputs + slots); tiles per wave = 8 * groups; cycles per tile "
           "per CU at a nominal 2.4 GHz, after the table fill (setup)\n");
    printf("| waves per workgroup | setup us | computed us (cyc/tile/CU) | table | half-table | recurrence |\n");
    printf("|---|---|---|---|---|---|\n");
    for (int waves : { 4, 8, 12, 16 })
    {
        const int ng = 200;
        std::vector<float> h0, h1, h2, h3, hz;
        const double z = run<1>(waves, 0, nblk, hz, 1);       // table fill + setup only
        const double t0 = run<0>(waves, ng, nblk, h0, 0);
        const double t1 = run<1>(waves, ng, nblk, h1, 1);
        const double t2 = run<2>(waves, ng, nblk, h2, 1);
        const double t3 = run<3>(waves, ng, nblk, h3, 0);
        const double tiles = (double)nblk * waves * ng * 8;
        auto same = [&](const std::vector<float>& h) { return std::memcmp(h0.data(), h.data(), h0.size() * 4) == 0; };
        auto cyc = [&](double ms) { return ms * 1e-3 * 2.4e9 / (tiles / 256.0); };   // cycles per tile per CU
        printf("| %d | %.1f | %.1f (%.2f) | %.1f (%.2f) %s | %.1f (%.2f) %s | %.1f (%.2f) %s |\n", waves, z * 1e3,
               t0 * 1e3, cyc(t0), t1 * 1e3, cyc(t1 - z), same(h1) ? "bit-exact" : "MISMATCH", t2 * 1e3, cyc(t2 - z),
               same(h2) ? "bit-exact" : "MISMATCH", t3 * 1e3, cyc(t3), same(h3) ? "bit-exact" : "MISMATCH");
        fflush(stdout);
    }
    return 0;
}
