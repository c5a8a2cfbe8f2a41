// The per-token state walk shared by the recurrent decode kernel and the fused decode kernel (gfx950, wave64).
//
// One workgroup of 512 threads (8 wave64) owns the 64 KiB fp32 state [V = 128][K = 128] of one (sequence, head).
// Lanes 32 h .. 32 h + 31 of wave w hold state row  16 p + 2 w + h  (p = 0..7) at columns  4 (l % 32) .. + 3:
// 8 f32x4 registers per lane; one wave instruction touches 2 full rows (1 KiB contiguous) and the workgroup 8 KiB
// contiguous per p.  A whole state in one workgroup with >= 8 waves, nontemporal loads and write-through stores
// (sc0 | sc1) is the measured best read-modify-write pattern on MI355X (6.2 TB/s against 5.1 TB/s for 4-wave
// workgroups with the default cache policy, and 5.4 TB/s for 8-wave workgroups on half a state).  Row reductions (S k, S q) run over 32 lanes: 4 DPP steps inside a row of 16 lanes and one
// swizzle across the two rows.
#pragma once
#include "common.h"

namespace kda355 {

constexpr int WK_THREADS = 512;
constexpr int WK_LOAD_AUX = 2;    // nt: streaming load
constexpr int WK_STORE_AUX = 17;     // sc0 | sc1: system-scope store, written through the L2
constexpr int WK_STORE_AUX_NT = 18;  // sc1 | nt: streaming store
// Store policy by the bytes of state a launch writes.  Write-through keeps the written states in the 256 MB MALL for
// the next step's reads; beyond that size they cannot stay there, and streaming stores write faster (measured on
// page pools: 537 MB of states per launch 214 -> 193 us, 268 MB 90 -> 107 us, so the switch sits between them).
constexpr long long WK_STREAM_BYTES = 384ll << 20;

// Sum over the 32 lanes of each half wave; every lane of the half receives the total.
__device__ __forceinline__ float sum32(float x) {
    x = sum16(x);
    // ds_swizzle bit mode: and 0x1f, or 0, xor 0x10 -> lane ^ 16 inside each group of 32
    return x + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));
}

struct Walker {
    int w, half, c;  // wave, half wave, column group (columns 4c .. 4c + 3)
    __device__ __forceinline__ explicit Walker(int tid) : w(tid >> 6), half((tid >> 5) & 1), c(tid & 31) {}
    __device__ __forceinline__ int row(int p) const { return 16 * p + 2 * w + half; }
    // byte offset of row p = voff() + p * 8 KiB: the lane part stays in one VGPR, the row step is an SGPR offset
    __device__ __forceinline__ int voff() const { return ((2 * w + half) * D + 4 * c) * 4; }
};
constexpr int WK_ROW_STEP = 16 * D * 4;


__device__ __forceinline__ __amdgpu_buffer_rsrc_t state_rsrc(const float* base) {
    return __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(base), (short)0, D * D * 4, 0x00020000);
}

// NP < 8: the workgroup holds rows 0 .. 16 NP - 1 of the block at `base` (a slice of a state), NP rows per lane.
template <int NP = 8>
__device__ __forceinline__ void load_state(const Walker& wk, const float* base, f32x4 (&st)[NP]) {
    const __amdgpu_buffer_rsrc_t rs = state_rsrc(base);
#pragma unroll
    for (int p = 0; p < NP; ++p)
        st[p] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, wk.voff(), p * WK_ROW_STEP, WK_LOAD_AUX));
}

// Wait for the state loads here rather than at the state's first use inside a token loop: the compiler's wait
// there would also run on every later iteration, where it drains that iteration's predecessor's state stores.
template <int NP = 8>
__device__ __forceinline__ void state_ready(f32x4 (&st)[NP]) {
#pragma unroll
    for (int p = 0; p < NP; ++p) asm volatile("" : "+v"(st[p]));
}

// valid = false stores nothing: the descriptor then covers 0 bytes and the hardware drops out-of-range buffer
// stores.  Keeping the store instructions unconditional keeps the compiler's memory-counter waits exact (a store
// under a branch makes it wait for every older access on the path without it).  NT selects the streaming policy at
// compile time: a run-time branch between the two policies costs the single-token decode 7 % (the stores can no
// longer start while the last rows are still being updated).
template <bool NT = false, int NP = 8>
__device__ __forceinline__ void store_state(const Walker& wk, float* base, const f32x4 (&st)[NP], bool valid = true) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(base), (short)0, valid ? 16 * NP * D * 4 : 0, 0x00020000);
#pragma unroll
    for (int p = 0; p < NP; ++p)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, st[p]), rs, wk.voff(), p * WK_ROW_STEP,
                                               NT ? WK_STORE_AUX_NT : WK_STORE_AUX);
}

// A buffer descriptor over `bytes` bytes at a wave-uniform base (the per-token operand rows).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(base), (short)0, bytes, 0x00020000);
}
// 4 bf16 at byte offset off of a row -> fp32
__device__ __forceinline__ void load_bf16x4(__amdgpu_buffer_rsrc_t rs, int off, float (&x)[4]) {
    const u32x2 b = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0));
    x[0] = bf2f(b.x & 0xffffu); x[1] = bf2f(b.x >> 16); x[2] = bf2f(b.y & 0xffffu); x[3] = bf2f(b.y >> 16);
}

// x * rsqrt(sum x^2 + 1e-6) over the 128 channels held 4 per lane by each half wave (kda/mi350x/reference.py:159-160).
__device__ __forceinline__ void rsqrt_norm4(float (&x)[4]) {
    const float s = sum32(x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3]);
    const float r = __frsqrt_rn(s + 1e-6f);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] *= r;
}

// v of row 16 p + 2 w + half from the lanes that hold it: lane c of each 16-lane row holds v[16 (c % 8) + 2 w + half]
// (vsrc); ds_swizzle bit mode (and 0x10, or p) reads lane p of the caller's 16-lane row.
template <int P>
__device__ __forceinline__ float v_of_row(float vsrc) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(vsrc), (P << 5) | 0x10));
}
// Lane c's source row for v_of_row: 16 (c % 8) + 2 w + half.
__device__ __forceinline__ int v_src_row(const Walker& wk) { return 16 * (wk.c & 7) + 2 * wk.w + wk.half; }

// One token of the gated delta rule on this lane's NP rows (8: a whole state per workgroup; fewer: a slice of 16 NP
// rows): S *= exp(g) along K; u = beta (v - S k); S += u k^T; o = scale * (S_decayed q + u (k . q)) (= scale * S_new q).
// dd = exp(g) of the lane's 4 key columns, vsrc = v at row v_src_row() of the slice (each row's v is broadcast from
// it; lanes with c % 8 >= NP hold any value).  Every lane of a half wave computes its rows' full sums; the return
// value is o at row 16 c + 2 w + half (meaningful on lanes c < NP).  Rows are reduced in groups of 4 to keep few
// values live.
// walk_token_kq: the same with k . q supplied by the caller (formed before the walk when the token's operands do not
// depend on the state).
template <int NP = 8>
__device__ __forceinline__ float walk_token_kq(f32x4 (&st)[NP], const float (&kk)[4], const float (&qq)[4],
                                               const float (&dd)[4], float vsrc, float bt, float kq, float scale, int c) {
    constexpr int GS = NP < 4 ? NP : 4;  // rows per group
    float vv[NP];
    vv[0] = v_of_row<0>(vsrc);
    if constexpr (NP > 1) vv[1] = v_of_row<1>(vsrc);
    if constexpr (NP > 2) { vv[2] = v_of_row<2>(vsrc); vv[3] = v_of_row<3>(vsrc); }
    if constexpr (NP > 4) {
        vv[4] = v_of_row<4>(vsrc); vv[5] = v_of_row<5>(vsrc); vv[6] = v_of_row<6>(vsrc); vv[7] = v_of_row<7>(vsrc);
    }
    float osel = 0.f;
#pragma unroll
    for (int g = 0; g < NP / GS; ++g) {
        float ak[GS], aq[GS];
#pragma unroll
        for (int i = 0; i < GS; ++i) {
            f32x4& s = st[GS * g + i];
            s.x *= dd[0]; s.y *= dd[1]; s.z *= dd[2]; s.w *= dd[3];
            ak[i] = s.x * kk[0] + s.y * kk[1] + s.z * kk[2] + s.w * kk[3];
            aq[i] = s.x * qq[0] + s.y * qq[1] + s.z * qq[2] + s.w * qq[3];
        }
#pragma unroll
        for (int i = 0; i < GS; ++i) { ak[i] = sum32(ak[i]); aq[i] = sum32(aq[i]); }
#pragma unroll
        for (int i = 0; i < GS; ++i) {
            f32x4& s = st[GS * g + i];
            const float u = bt * (vv[GS * g + i] - ak[i]);
            const float o = scale * (aq[i] + u * kq);
            osel = (c == GS * g + i) ? o : osel;
            s.x += u * kk[0]; s.y += u * kk[1]; s.z += u * kk[2]; s.w += u * kk[3];
        }
    }
    return osel;
}
template <int NP = 8>
__device__ __forceinline__ float walk_token(f32x4 (&st)[NP], const float (&kk)[4], const float (&qq)[4],
                                            const float (&dd)[4], float vsrc, float bt, float scale, int c) {
    const float kq = sum32(kk[0] * qq[0] + kk[1] * qq[1] + kk[2] * qq[2] + kk[3] * qq[3]);
    return walk_token_kq<NP>(st, kk, qq, dd, vsrc, bt, kq, scale, c);
}

// Sum over the 64 lanes of a wave, returned wave-uniform.
__device__ __forceinline__ float sum64(float x) {
    x = sum32(x);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0)) +
           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
}

}  // namespace kda355
