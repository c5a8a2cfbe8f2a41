// Device helpers shared by the kda355 kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/kda355.h"

namespace kda355 {

constexpr int D = KDA355_HEAD_DIM;
constexpr int CH = KDA355_CHUNK;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// bf16 bits <-> fp32 (the bf16 value widened exactly)
__device__ __forceinline__ float bf2f(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
// fp32 -> bf16 bits, round to nearest even (gfx950 converts in hardware: v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t f2bf(float x) {
    const __bf16 b = (__bf16)x;
    return (uint32_t)__builtin_bit_cast(uint16_t, b);
}

// two fp32 -> packed bf16 pair (x0 in the low half), round to nearest even: one v_cvt_pk_bf16_f32
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f2bf2(float x0, float x1) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x0, x1}, bf16x2_t));
}

// XCD-aware task order.  Workgroup b of a launch runs on XCD b % 8 (round-robin dispatch over the 8 XCDs of an
// MI355X); giving each XCD a contiguous range of (sequence, head) tasks keeps the workgroups that touch neighbouring
// data (neighbouring 64 KiB state blocks, or the row blocks of one state) on one XCD and its L2.
// Exact bijection of [0, total): XCD x owns [x (total / 8) + min(x, total % 8), ...) of size total / 8 + (x < total % 8).
__device__ __forceinline__ int xcd_task(int b, int total) {
    const int x = b & 7, q = total >> 3, r = total & 7;
    return x * q + (x < r ? x : r) + (b >> 3);
}

// A wave-uniform address taken through readfirstlane: the compiler may otherwise compute uniform 64-bit address
// arithmetic in VGPRs (v_lshl_add_u64), and a buffer descriptor built from a VGPR base becomes a waterfall loop.
__device__ __forceinline__ void* uniform_ptr(const void* p) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
}

// DPP lane moves inside a row of 16 lanes (quad_perm / row_half_mirror / row_mirror).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
// Sum over each group of 16 consecutive lanes; every lane of the group receives the total.
__device__ __forceinline__ float sum16(float x) {
    x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
    x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
    x += dpp<0x141>(x);  // row_half_mirror
    x += dpp<0x140>(x);  // row_mirror
    return x;
}

// through the hardware reciprocal (v_rcp_f32, within 1 ulp): an IEEE division is a sequence of about ten instructions
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// Workgroup barrier that orders LDS only: __syncthreads() also waits for every outstanding global load and store
// (vmcnt(0)), which would stall on loads issued for later phases.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Thread-local error text for the C ABI.
void set_error(const char* fmt, ...);

}  // namespace kda355

#define KDA_CHECK_ARG(cond, ...)                 \
    do {                                         \
        if (!(cond)) {                           \
            ::kda355::set_error(__VA_ARGS__);    \
            return KDA355_EINVAL;                \
        }                                        \
    } while (0)
