// esda_device.h -- device helpers shared by the HIP kernels of libesda.so (gfx950 only):
// vector types, the LDS DMA and barrier primitives, a cross-lane-group max, compile-time
// unrolling, an fp32 sincos and bf16 unpacking.  Each includer gets its own copies
// (anonymous namespace).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>
#include <utility>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef short short8v __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// Max over the four 16-lane groups of a wave (lanes l, l^16, l^32, l^48) without
// touching LDS.  v_permlane16_swap_b32 a, b exchanges the odd 16-lane rows of a with
// the even rows of b (v_permlane32_swap_b32: the upper half of a with the lower half of
// b); with a = b = x, max(a, b) is then the max over row pairs, and over halves.  The
// swaps are written in assembly because this toolchain's builtins hand back the first
// register for both results, which silently drops the partner row from the max.
__device__ __forceinline__ float wave_max_across_groups(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
    unsigned a = __builtin_bit_cast(unsigned, x), b = a;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    x = fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    a = __builtin_bit_cast(unsigned, x);
    b = a;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
#else
    return x;
#endif
}

// Sum over the four 16-lane groups of a wave (lanes l, l^16, l^32, l^48), by the same
// swaps; integer adds, so the sum is exact and the same in all four lanes.
__device__ __forceinline__ unsigned wave_sum_across_groups(unsigned x) {
#if defined(__HIP_DEVICE_COMPILE__)
    unsigned a = x, b = x;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    a += b;
    b = a;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return a + b;
#else
    return x;
#endif
}

// The running max is only raised (and O rescaled) once a score exceeds it by this
// much in log2 units; until then probabilities may reach 2^8 before normalisation,
// far from fp32 / bf16 limits, and the final division by l is unchanged.
constexpr float kRescaleSlack = 8.0f;

// x *= c for a value that lives in an accumulation register (AGPR): read, multiply and
// write back in place.  With a plain multiply of the PV accumulators the compiler keeps
// VGPR copies of all of them, refreshed at every stage, for a rescale that is rare.
// (The MFMAs that next read x come dozens of instructions later, past any wait-state
// requirement of an AGPR write.)
__device__ __forceinline__ void acc_scale(float &x, float c) {
#if defined(__HIP_DEVICE_COMPILE__)
    float t;
    asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32_e32 %1, %2, %1\n\tv_accvgpr_write_b32 %0, %1"
                 : "+a"(x), "=&v"(t)
                 : "v"(c));
#else
    x *= c;
#endif
}

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8], vmcnt[5:4] at [15:14]).
#define ESDA_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))

// Workgroup barrier for LDS hand-offs.  __syncthreads() would also drain every
// outstanding global load (vmcnt(0)), which would empty the DMA ring each stage; the
// ring's own vmcnt waits precede this barrier instead.  The memory clobber keeps the
// compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#endif
}

// One 64-lane x 16-byte LDS DMA (global_load_lds_dwordx4; non-temporal unless NT is
// false, for data other workgroups read again): lane l's 16 bytes from `src` land at LDS
// byte address lds + 16*l.  Issued from inline assembly so
// that the compiler does not track it: the ring accounts for these loads itself
// (ESDA_WAIT_VM before each stage), and compiler-inserted waits would drain the ring.
// M0 carries the LDS base; nothing else in these kernels uses M0.
// (The guard keeps the gfx950 assembly out of hipcc's host pass.)
template <bool NT = true>
__device__ __forceinline__ void lds_dma16(const void *src, unsigned lds) {
#if defined(__HIP_DEVICE_COMPILE__)
    const unsigned base = __builtin_amdgcn_readfirstlane(lds);  // wave-uniform by construction
    if constexpr (NT)
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(base) : "memory");
    else
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(base) : "memory");
#endif
}

// Same DMA with a wave-uniform 64-bit base in SGPRs and a per-lane 32-bit byte offset:
// interior stages advance the base with scalar adds and reuse the lane offsets.
template <bool NT = true>
__device__ __forceinline__ void lds_dma16_s(const void *sbase, unsigned voff, unsigned lds) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uintptr_t a = (uintptr_t) sbase;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned) a);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned) (a >> 32));
    const uint64_t sb = ((uint64_t) hi << 32) | lo;
    const unsigned base = __builtin_amdgcn_readfirstlane(lds);
    if constexpr (NT)
        asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sb), "s"(base) : "memory");
    else
        asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sb), "s"(base) : "memory");
#endif
}

// A wave-uniform 64-bit address as a scalar pair (the base operand of lds_dma16_o).
__device__ __forceinline__ uint64_t sbase64(const void *p) {
    const uintptr_t a = (uintptr_t) p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned) a);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned) (a >> 32));
    return ((uint64_t) hi << 32) | lo;
}

// The DMA of lds_dma16_s with the instruction's immediate offset OFF (0 .. 3072 here),
// which gfx950 adds to both addresses: lane l's 16 bytes come from sbase + voff + OFF and
// land at LDS byte m0 + OFF + 16 l.  M0 is set to lds + MOFF by one scalar add, so rows
// that are OFF apart in memory but spaced otherwise in LDS (padded blocks) share one
// scalar base: a row costs one scalar instruction beside its DMA.
template <int OFF, int MOFF, bool NT = true>
__device__ __forceinline__ void lds_dma16_o(uint64_t sbase, unsigned voff, unsigned lds) {
#if defined(__HIP_DEVICE_COMPILE__)
    static_assert(OFF >= 0 && OFF < 4096, "the immediate offset is a 12-bit field here");
    if constexpr (NT)
        asm volatile("s_add_u32 m0, %2, %3\n\tglobal_load_lds_dwordx4 %0, %1 offset:%4 nt"
                     ::"v"(voff), "s"(sbase), "s"(lds), "i"(MOFF), "i"(OFF) : "memory");
    else
        asm volatile("s_add_u32 m0, %2, %3\n\tglobal_load_lds_dwordx4 %0, %1 offset:%4"
                     ::"v"(voff), "s"(sbase), "s"(lds), "i"(MOFF), "i"(OFF) : "memory");
#endif
}

// One 4-byte LDS DMA per active lane (global_load_lds_dword): active lane l's 4 bytes land
// at LDS byte address lds + 4*l.  Counted by the ring like lds_dma16.
__device__ __forceinline__ void lds_dma4(const void *src, unsigned lds) {
#if defined(__HIP_DEVICE_COMPILE__)
    const unsigned base = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(base) : "memory");
#endif
}

// A value that is the same in every lane, as a scalar.
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

__device__ __forceinline__ unsigned lds_addr(const void *p) {
    return (unsigned) (uintptr_t) (const __attribute__((address_space(3))) void *) p;
}

// Calls f(std::integral_constant<int, 0>) .. f(std::integral_constant<int, N-1>): a
// guaranteed full unroll in which the index is a compile-time constant.
template <class F, int... I>
__device__ __forceinline__ void unroll_impl(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void unroll(F &&f) {
    unroll_impl(f, std::make_integer_sequence<int, N>{});
}

// Cody-Waite split of pi/2 (hi + mid + lo, each the nearest fp32 to what remains).
constexpr float kTwoOverPi = 0.636619746685028076171875f;     // fp32(2/pi)
constexpr float kPio2Hi = 1.57079637050628662109375f;         // fp32(pi/2)
constexpr float kPio2Mid = -4.37113882867379300296306610107421875e-8f;
constexpr float kPio2Lo = -1.715124510005881916757519826222e-15f;

// cos and sin of an fp32 angle |a| < 2^20.  Reduction a = n*pi/2 + r in three FMA
// steps (the first is exact: n*hi is a multiple of 2^-23 within 1 of a), then Taylor
// polynomials on |r| <= pi/4 (truncation error < 2e-9), then the quadrant n mod 4.
// Absolute error is a few 1e-8, far inside the bf16 rounding applied to the results.
__device__ __forceinline__ void sincos_f32(float a, float &s, float &c) {
    const float n = __builtin_rintf(a * kTwoOverPi);
    float r = __builtin_fmaf(-n, kPio2Hi, a);
    r = __builtin_fmaf(-n, kPio2Mid, r);
    r = __builtin_fmaf(-n, kPio2Lo, r);
    const float r2 = r * r;
    float ps = __builtin_fmaf(r2, 1.0f / 362880.0f, -1.0f / 5040.0f);
    ps = __builtin_fmaf(r2, ps, 1.0f / 120.0f);
    ps = __builtin_fmaf(r2, ps, -1.0f / 6.0f);
    const float sr = __builtin_fmaf(r * r2, ps, r);
    float pc = __builtin_fmaf(r2, -1.0f / 3628800.0f, 1.0f / 40320.0f);
    pc = __builtin_fmaf(r2, pc, -1.0f / 720.0f);
    pc = __builtin_fmaf(r2, pc, 1.0f / 24.0f);
    pc = __builtin_fmaf(r2, pc, -0.5f);
    const float cr = __builtin_fmaf(r2, pc, 1.0f);
    const int q = (int) n & 3;
    s = (q & 1) ? cr : sr;
    c = (q & 1) ? sr : cr;
    if (q & 2) s = -s;
    if ((q + 1) & 2) c = -c;
}

__device__ __forceinline__ float bf16_lo(unsigned w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(unsigned w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

}  // namespace
