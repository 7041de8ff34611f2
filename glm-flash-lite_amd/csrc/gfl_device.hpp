// Device helpers shared by the gfx950 kernels: EXL3 trellis decode, fp16 rounding points, wave-level Hadamard-128.
//
// Trellis format (kernels/cpu_avx2/ft_core.h:28-83 of the reference): a 16x16 tile is a circular 256*K-bit stream,
// MSB-first inside little-endian 32-bit words; weight t takes the 16-bit state ending at bit (t+1)*K, hashes it as
// bytesum(state * 0x83DCD12D mod 2^32) and maps it to fp16 with one rounding of fma(1024 + sum, KINV, KBIAS).
// Stream index t*8+j sits at tile row {r0, r0+1, r0+8, r0+9}[j%4] (r0 = 2*(t%4)), column t/4 + 8*(j>=4).
//
// Lane layout used everywhere: lane l = 16*q + n decodes the four consecutive stream indices
// 32*(n%8) + 8*q + 4*(n/8) + {0,1,2,3}, i.e. column n, rows 2q + {0,1,8,9} of the tile. Those four weights are
// exactly the MFMA 16x16x16 B-operand slice of lane l when the K index is 4q + j.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace gfl {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr uint32_t MUL1 = 0x83DCD12Du;
constexpr float HADF = 0.088388347648f;
constexpr uint16_t KINV_BITS = 0x1eee, KBIAS_BITS = 0xc931;

// Per-lane decode constants: byte offsets of the two words holding the lane's 3K+16-bit window inside a tile, and the
// funnel shift that puts the window's last bit at bit 0.
struct LaneDec
{
    uint32_t o0, o1, sh;
};

__host__ __device__ inline LaneDec lane_dec(int lane, int K)
{
    const int q = lane >> 4, n = lane & 15;
    const int S = 32 * (n & 7) + 8 * q + 4 * (n >> 3);  // first stream index of the lane's run
    const int e = (S + 4) * K;                           // end (exclusive) of the run's window, in stream bits
    const int words = 8 * K;
    const int wa = (e - 33) >= 0 ? (e - 33) / 32 : -1;  // floor((e-33)/32): e - 32*wa in [33, 64]
    LaneDec d;
    d.sh = (uint32_t)(64 - (e - 32 * wa));
    d.o0 = (uint32_t)(4 * ((wa + words) % words));
    d.o1 = (uint32_t)(4 * ((wa + 1 + words) % words));
    return d;
}

__device__ inline uint32_t ld_u32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// Pointers into global memory in the global address space. Addresses read from the layer table are otherwise generic
// to the compiler, and a generic (flat) load counts on both the vector-memory and the LDS counters, so the compiler
// can only wait for it with vmcnt(0), which also waits for every load issued before it (prefetches and LDS-direct
// loads included). The table holds device-memory addresses only.
template <typename T>
using gptr = const __attribute__((address_space(1))) T*;

template <typename T>
__device__ __forceinline__ gptr<T> gaddr(uint64_t a)
{
    return (gptr<T>)a;
}

// the 16 bytes at element i of a global pointer (loaded as a native vector: HIP's uint4 has no copy from another
// address space)
template <typename T>
__device__ __forceinline__ uint4 gld16(gptr<T> p, long i)
{
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = *reinterpret_cast<gptr<u32x4>>(p + i);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// A pointer that is the same in every lane of the wave, moved to scalar registers. __builtin_amdgcn_readfirstlane
// takes and returns a 32-bit int, so the two halves of the 64-bit address go through it separately.
__device__ inline const uint8_t* uniform_ptr(const uint8_t* p)
{
    const uint64_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
    return reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
}

// four 16-bit states -> their four fp16 codebook weights
__device__ inline half4 codebook4(uint32_t st0, uint32_t st1, uint32_t st2, uint32_t st3)
{
    const uint32_t p0 = st0 * MUL1, p1 = st1 * MUL1, p2 = st2 * MUL1, p3 = st3 * MUL1;
    // sum of the product bytes on top of 0x6400 = fp16 bits of (1024 + sum); the hi variant lands in bits 16..31
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
    // one fp16 rounding of an exact product-sum (v_pk_fma_f16): equals round16(fma_f32(1024+s, KINV, KBIAS))
    const half2v w01 = __builtin_elementwise_fma(a, kinv2, kbias2);
    const half2v w23 = __builtin_elementwise_fma(b, kinv2, kbias2);
    half4 r = { w01[0], w01[1], w23[0], w23[1] };
    return r;
}

// four consecutive states -> four fp16 codebook weights, packed {w0,w1}, {w2,w3}
template <int K>
__device__ inline half4 decode4(uint32_t hi, uint32_t lo, uint32_t sh)
{
    const uint32_t R = __builtin_amdgcn_alignbit(hi, lo, sh);
    return codebook4(__builtin_amdgcn_ubfe(R, 3 * K, 16), __builtin_amdgcn_ubfe(R, 2 * K, 16),
                     __builtin_amdgcn_ubfe(R, K, 16), __builtin_amdgcn_ubfe(R, 0, 16));
}

// fp32 -> fp16 (round to nearest even, subnormals kept) as an opaque conversion. The reference rounds every product
// to fp32 before rounding it to fp16 (e.g. r16(y * HAD), ft_core.h:102,109); left to itself the compiler fuses
// fptrunc(a*b) into one v_fma_mixlo_f16, which rounds once and differs at fp16 ties.
__device__ inline uint32_t f2h_bits(float x)
{
    uint32_t h;
    asm("v_cvt_f16_f32 %0, %1" : "=v"(h) : "v"(x));
    return h & 0xFFFFu;
}

// two fp32 -> their fp16 bits packed lo | hi << 16, each rounded like f2h_bits (the high half through the SDWA form,
// which keeps the low half)
__device__ inline uint32_t f2h2_bits(float lo, float hi)
{
    uint32_t h;
    asm("v_cvt_f16_f32 %0, %1\n\tv_cvt_f16_f32_sdwa %0, %2 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD"
        : "=&v"(h)
        : "v"(lo), "v"(hi));
    return h;
}

__device__ inline float r16(float x)
{
    uint32_t h;
    float r;
    asm("v_cvt_f16_f32 %0, %1" : "=v"(h) : "v"(x));
    asm("v_cvt_f32_f16 %0, %1" : "=v"(r) : "v"(h));
    return r;
}

// Value of lane L ^ W (W = 1..32) without the LDS crossbar: DPP quad permutes, mirrors and rotates inside 16-lane
// rows (xor 4 = half-row mirror then xor 3, xor 8 = rotate the row by 8), gfx950's permlane swaps across rows.
template <int W>
__device__ __forceinline__ float lane_xor(float v)
{
    const int iv = __float_as_int(v);
    if constexpr (W == 1) return __int_as_float(__builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xF, 0xF, true));
    if constexpr (W == 2) return __int_as_float(__builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xF, 0xF, true));
    if constexpr (W == 4)
    {
        const int t = __builtin_amdgcn_update_dpp(0, iv, 0x141, 0xF, 0xF, true);   // row_half_mirror: L ^ 7
        return __int_as_float(__builtin_amdgcn_update_dpp(0, t, 0x1B, 0xF, 0xF, true));   // quad_perm 3210: ^ 3
    }
    if constexpr (W == 8) return __int_as_float(__builtin_amdgcn_update_dpp(0, iv, 0x128, 0xF, 0xF, true));   // row_ror:8
    if constexpr (W == 16)
    {
        // odd rows of the first operand <-> even rows of the second: {rows 0,0,2,2 ; rows 1,1,3,3}
        const auto r = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
        return __int_as_float((threadIdx.x & 16) ? r[0] : r[1]);
    }
    if constexpr (W == 32)
    {
        // upper half of the first operand <-> lower half of the second: {lanes 0..31 twice ; 32..63 twice}
        const auto r = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
        return __int_as_float((threadIdx.x & 32) ? r[0] : r[1]);
    }
}

// Wave-level Hadamard-128 in the reference's butterfly order (had128, ft_core.h:89-94): lane L holds elements L and
// L+64; stages w = 1..32 cross lanes, w = 64 stays in the lane. Every element sees the same add/sub sequence.
template <int W>
__device__ __forceinline__ void fwht_stage(float& v0, float& v1, int L)
{
    const float p0 = lane_xor<W>(v0), p1 = lane_xor<W>(v1);
    if (L & W) { v0 = p0 - v0; v1 = p1 - v1; }
    else { v0 = v0 + p0; v1 = v1 + p1; }
}

__device__ inline void fwht128(float& v0, float& v1)
{
    const int L = threadIdx.x & 63;
    fwht_stage<1>(v0, v1, L);
    fwht_stage<2>(v0, v1, L);
    fwht_stage<4>(v0, v1, L);
    fwht_stage<8>(v0, v1, L);
    fwht_stage<16>(v0, v1, L);
    fwht_stage<32>(v0, v1, L);
    const float a = v0, c = v1;
    v0 = a + c;
    v1 = a - c;
}

// Element r (0..127) of a 128-block (= one group of 8 tile rows) -> its position in the GEMM input layout
// [block][q][tile row][jj]: row rho = r % 16 of tile row r / 16 is MFMA k-slot jj = (rho&1) + 2*(rho>>3) of lane group
// q = (rho&7)>>1, so the 4 k-slots of two consecutive tile rows of one q are 8 contiguous fp16.
__device__ inline int gp_perm_pos(int b, int r)
{
    const int tr = r >> 4, rho = r & 15;
    const int jj = (rho & 1) + 2 * (rho >> 3), q = (rho & 7) >> 1;
    return b * 128 + q * 32 + tr * 4 + jj;
}

// Elements 8li..8li+7 of block b in the GEMM input layout gp_perm_pos: pairs (2q, 2q + 1) are adjacent, at
// b * 128 + q * 32 + (li >> 1) * 4 + 2 * (li & 1)
__device__ __forceinline__ void gp_store_row(uint16_t* dst, int b, int li, const uint32_t (&o)[4])
{
    uint16_t* d0 = dst + b * 128 + (li >> 1) * 4 + 2 * (li & 1);
#pragma unroll
    for (int q = 0; q < 4; ++q) *reinterpret_cast<uint32_t*>(d0 + q * 32) = o[q];
}

__device__ inline float h2f_bits(uint16_t h) { __half x; __builtin_memcpy(&x, &h, 2); return __half2float(x); }

// Hadamard-128 on one 16-lane row of the wave, 8 elements per lane: lane i of the row holds elements 8i..8i+7.
// Stages h = 1, 2, 4 pair elements inside the lane, h = 8..64 pair lane i with i ^ (h / 8); every element sees the
// same add/sub sequence as had128 (ft_core.h:89-94): the lower element of a pair becomes a + b, the upper a - b.
// Across lanes the upper lane keeps its own value minus its partner's, the negated a - b, so that every lane does the
// same one instruction per element (an fma with its partner's value by DPP and a per-lane +-1); the negations add up
// to a per-lane sign (-1)^popcount(i), which fwht128_row returns. Negation commutes with rounding, so sign * v is
// exactly had128's result, and callers fold the sign into their next product.
//
// v[k] += sg * (v[k] of the partner lane) for the 8 elements, as v_fmac_f32 with a DPP source (the compiler keeps a
// separate DPP move there). The leading s_nop covers the VALU-write -> DPP-read hazard on the values written just
// before; inside a block each element's DPP read comes 8 instructions after that element's previous write.
#define GFL_FMAC8(CTRL, S0, S1, S2, S3, S4, S5, S6, S7)                                                          \
    "s_nop 1\n\t"                                                                                                      \
    "v_fmac_f32_dpp %0, " S0 ", %8 " CTRL "\n\tv_fmac_f32_dpp %1, " S1 ", %8 " CTRL "\n\t"                           \
    "v_fmac_f32_dpp %2, " S2 ", %8 " CTRL "\n\tv_fmac_f32_dpp %3, " S3 ", %8 " CTRL "\n\t"                           \
    "v_fmac_f32_dpp %4, " S4 ", %8 " CTRL "\n\tv_fmac_f32_dpp %5, " S5 ", %8 " CTRL "\n\t"                           \
    "v_fmac_f32_dpp %6, " S6 ", %8 " CTRL "\n\tv_fmac_f32_dpp %7, " S7 ", %8 " CTRL
#define GFL_DPP_ALL " row_mask:0xf bank_mask:0xf bound_ctrl:1"

template <int W>
__device__ __forceinline__ void fwht_row_stage(float (&v)[8], int L)
{
    const float sg = (L & W) ? -1.0f : 1.0f;
    if constexpr (W == 1)
        asm(GFL_FMAC8("quad_perm:[1,0,3,2]" GFL_DPP_ALL, "%0", "%1", "%2", "%3", "%4", "%5", "%6", "%7")
            : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])
            : "v"(sg));
    else if constexpr (W == 2)
        asm(GFL_FMAC8("quad_perm:[2,3,0,1]" GFL_DPP_ALL, "%0", "%1", "%2", "%3", "%4", "%5", "%6", "%7")
            : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])
            : "v"(sg));
    else if constexpr (W == 8)
        asm(GFL_FMAC8("row_ror:8" GFL_DPP_ALL, "%0", "%1", "%2", "%3", "%4", "%5", "%6", "%7")
            : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])
            : "v"(sg));
    else
    {
        static_assert(W == 4, "row stages are 1, 2, 4, 8");
        // lane L ^ 4 = half-row mirror (L ^ 7) of quad_perm 3210 (L ^ 3): the mirrored copies first, 8 moves apart
        // from their DPP reads
        float t[8];
        asm("s_nop 1\n\t"
            "v_mov_b32_dpp %0, %8 row_half_mirror" GFL_DPP_ALL "\n\tv_mov_b32_dpp %1, %9 row_half_mirror" GFL_DPP_ALL "\n\t"
            "v_mov_b32_dpp %2, %10 row_half_mirror" GFL_DPP_ALL "\n\tv_mov_b32_dpp %3, %11 row_half_mirror" GFL_DPP_ALL "\n\t"
            "v_mov_b32_dpp %4, %12 row_half_mirror" GFL_DPP_ALL "\n\tv_mov_b32_dpp %5, %13 row_half_mirror" GFL_DPP_ALL "\n\t"
            "v_mov_b32_dpp %6, %14 row_half_mirror" GFL_DPP_ALL "\n\tv_mov_b32_dpp %7, %15 row_half_mirror" GFL_DPP_ALL
            : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]), "=&v"(t[4]), "=&v"(t[5]), "=&v"(t[6]), "=&v"(t[7])
            : "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]), "v"(v[7]));
        asm(GFL_FMAC8("quad_perm:[3,2,1,0]" GFL_DPP_ALL, "%9", "%10", "%11", "%12", "%13", "%14", "%15", "%16")
            : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])
            : "v"(sg), "v"(t[0]), "v"(t[1]), "v"(t[2]), "v"(t[3]), "v"(t[4]), "v"(t[5]), "v"(t[6]), "v"(t[7]));
    }
}
#undef GFL_FMAC8
#undef GFL_DPP_ALL

// Returns the lane's sign: the transform is sign * v.
__device__ inline float fwht128_row(float (&v)[8])
{
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (!(k & h))
            {
                const float a = v[k], b = v[k + h];
                v[k] = a + b;
                v[k + h] = a - b;
            }
    const int L = threadIdx.x & 15;
    fwht_row_stage<1>(v, L);
    fwht_row_stage<2>(v, L);
    fwht_row_stage<4>(v, L);
    fwht_row_stage<8>(v, L);
    return (__builtin_popcount(L) & 1) ? -1.0f : 1.0f;
}

__device__ __forceinline__ float h2f_lane(uint4 v, int k)
{
    const uint32_t w = k < 2 ? v.x : k < 4 ? v.y : k < 6 ? v.z : v.w;
    return h2f_bits((uint16_t)(w >> (16 * (k & 1))));
}

// out_block (ft_core.h:105-110) after its leading r16: v = the lane's 8 fp16-valued inputs, sc its 8 fp16 scales
__device__ inline void out_block_row_rounded(float (&v)[8], uint4 sc)
{
    const float sh = fwht128_row(v) * HADF;   // (sign * v) * HADF == v * (sign * HADF), bit for bit
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = r16(v[k] * sh * h2f_lane(sc, k));
}

// out_block (ft_core.h:105-110) on a 16-lane row: v = the lane's 8 fp32 outputs, sc its 8 fp16 scales
__device__ inline void out_block_row(float (&v)[8], uint4 sc)
{
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = r16(v[k]);
    out_block_row_rounded(v, sc);
}

// out_block from outputs stored already rounded to fp16 (raw = the lane's 8 fp16 values): the same results as
// out_block_row on the fp32 outputs, whose first step is that rounding
__device__ inline void out_block_row_h(float (&v)[8], uint4 raw, uint4 sc)
{
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = h2f_lane(raw, k);
    out_block_row_rounded(v, sc);
}

// prep_block (ft_core.h:97-102) on a 16-lane row up to its last rounding: v holds the lane's 8 fp32 inputs and sc its
// 8 fp16 scales; on return v = the fp32 products (H v) * HADF, each still to be rounded to fp16
__device__ inline void prep_block_row_fp(float (&v)[8], uint4 sc)
{
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = v[k] * h2f_lane(sc, k);
    const float sh = fwht128_row(v) * HADF;
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = v[k] * sh;
}

// the same from 8 fp16 inputs x (16 bytes); x * suh of two fp16 values is exact in fp32
__device__ inline void prep_block_row_p(float (&v)[8], uint4 x, uint4 sc)
{
    const uint32_t xw[4] = { x.x, x.y, x.z, x.w }, sw[4] = { sc.x, sc.y, sc.z, sc.w };
#pragma unroll
    for (int k = 0; k < 8; ++k)
        v[k] = h2f_bits((uint16_t)(xw[k >> 1] >> (16 * (k & 1)))) * h2f_bits((uint16_t)(sw[k >> 1] >> (16 * (k & 1))));
    const float sh = fwht128_row(v) * HADF;
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = v[k] * sh;
}

// prep_block with the 8 fp16 results packed in pairs: o[i] = elements 2i | 2i + 1 << 16
__device__ inline void prep_block_row_fh(uint32_t (&o)[4], float (&v)[8], uint4 sc)
{
    prep_block_row_fp(v, sc);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f2h2_bits(v[2 * i], v[2 * i + 1]);
}

__device__ inline void prep_block_row_h(uint32_t (&o)[4], uint4 x, uint4 sc)
{
    float v[8];
    prep_block_row_p(v, x, sc);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f2h2_bits(v[2 * i], v[2 * i + 1]);
}

// prep_block (ft_core.h:97-102) on lane-held elements L, L+64
__device__ inline void prep_block_wave(float& v0, float& v1, float s0, float s1)
{
    v0 = v0 * s0;
    v1 = v1 * s1;
    fwht128(v0, v1);
    v0 = r16(v0 * HADF);
    v1 = r16(v1 * HADF);
}

// out_block (ft_core.h:105-110)
__device__ inline void out_block_wave(float& v0, float& v1, float s0, float s1)
{
    v0 = r16(v0);
    v1 = r16(v1);
    fwht128(v0, v1);
    v0 = r16(v0 * HADF * s0);
    v1 = r16(v1 * HADF * s1);
}

// silu(g) * u with exllamav3's clamp (act_mul, ft_core.h:123-132), given x = silu(g) = g / (1 + expf(-g))
__device__ inline float act_mul_s(float x, float u, float limit)
{
    if (limit != 0.0f)
    {
        u = fminf(fmaxf(u, -limit), limit);
        x = fminf(x, limit);
    }
    return x * u;
}

// the same with silu(g) from the context's table, indexed by the fp16 bits of g (g is fp16-valued)
__device__ inline float act_mul(float g, float u, float limit, const float* __restrict__ silu_tab)
{
    return act_mul_s(silu_tab[f2h_bits(g) & 0xFFFFu], u, limit);
}

}  // namespace gfl
