// Chunked KDA prefill on gfx950 (chunk 64, head dim 128): host plan and one fused chunk kernel.
//
// Math (per sequence n, head h, chunk of c <= 64 tokens; Gamma = inclusive cumsum of the log-decay g over the chunk,
// per key channel; S the fp32 state, K-major [k][v] in the formulas, V-major [v][k] in memory):
//     A_kk = strict_tril(diag(beta) (K e^{Gamma}) (K e^{-Gamma})^T),   A_qk = tril((Q e^{Gamma}) (K e^{-Gamma})^T)
//     W = (I + A_kk)^-1 diag(beta) K e^{Gamma},   U = (I + A_kk)^-1 diag(beta) V
//     V' = U - W S;   O = scale (Q e^{Gamma} S + A_qk V');   S <- diag(e^{Gamma_c}) S + (K e^{Gamma_c - Gamma})^T V'
// This is the token recurrence of kda/mi350x/reference.py:85-91 regrouped per chunk (the chunked WY form; the same
// operator as kda/b200/csrc/w3/base/tiny/kda_tiny.cu:5-10 and vLLM's qg / w / u / kg_t / decay decomposition,
// kda/mi350x/benchmark/baselines/prefill/vllm_reference/kda_chunk.py:73-76, 97-108).
//
// One workgroup of 512 threads (8 wave64) walks the chunks of one (sequence, head) and keeps everything of a chunk
// on chip: the only HBM traffic is q, k, v, g, beta in, o out, and the state in / out / checkpoints.  The next
// chunk's inputs are prefetched into registers while the current chunk is processed.  Per chunk:
//   P0  raw rows -> LDS (gate), row norms (DPP)          thread (r = tid / 8, channels 16 (tid % 8) .. + 15)
//   P1  in-chunk gate cumsum, 4 segments of 16 rows      thread (channel tid % 128, segment tid / 128)
//   P2  per-element factors fi = e^{Gamma_i - Gamma_m}, fj = 1 / fi with m the middle row of the 16-row block,
//       and the per-channel block factors (a, b, x, y, decay) -- two exponentials per element
//   P4  Gram tiles on MFMA: the four diagonal 16 x 16 blocks from bf16 hi + lo operands (3 MFMAs: hi.hi + hi.lo +
//       lo.hi; their gated operands span e^{+-8|g|}), the six off-diagonal blocks from fp16 operands <= 1 (the
//       reference point is the last row before the row block); each diagonal wave then inverts its block,
//       (I + L_II)^-1 by forward substitution in fp32, while the off-diagonal waves finish
//   P5  Q e^Gamma, K e^{Gamma_c - Gamma} and beta V to LDS in the walk's operand layouts
//   P6  W and U by block forward substitution on MFMA: X_I = T_II (B_I - sum_{J<I} A_IJ X_J); wave w owns key
//       channels [16w, 16w+16) of W and value columns [16w, 16w+16) of U, so no wave waits for another
//   P7  the walk: wave w keeps the 128 x 16 slice S[:, 16w:16w+16] in fp32 registers (MFMA C layout) for the whole
//       sequence; V' = U - W S, O = scale (Q~ S + A_qk V'), S = diag(decay) S + Kd^T V' (16x16x32 f16 MFMAs whose B
//       operands come straight from the accumulators: the LDS operands are stored with the matching permutation of
//       each 32-block, position 8g + 4h + e <-> index 16h + 4g + e)
// Precision: MFMA operands are fp16 (11-bit significand) except the diagonal Gram blocks (bf16 hi/lo); fp32
// accumulation; the state is fp32 and is rounded to fp16 only as the B operand of W S and Q~ S.  Range: fp16 holds
// |x| < 65504 (state, U, T entries); the diagonal blocks need |Gamma_i - Gamma_m| <= 72 over 8 tokens, so every
// per-token log-decay is raised to KDA355_MIN_LOG_DECAY (-9) if it is below (clamp_decay).
#include <algorithm>
#include <functional>
#include <numeric>
#include <queue>
#include <vector>

#include "common.h"

namespace kda355 {
namespace {

constexpr int PF_THREADS = 512;

// LDS layout (bytes).  Region A: gate / Gamma fp32 [64][132], then k^ fi fp32 [64][132].  Region B: q^ fi fp32
// [64][132], then Q~ fp16 [64][136] and W fp16 [64][136].  Region C: k^ fj fp32 [64][132], then Kd^T fp16
// [128][72].  The row paddings keep the scattered two-byte stores of the layouts and the column reads free of bank
// conflicts and every MFMA fragment at a constant offset from its lane's base.  On gfx950 the 16-byte fragment reads
// of these rows still take two LDS passes (SQ_LDS_BANK_CONFLICT); swizzled rows that read in one pass measured no
// faster, since the kernel's phases wait on VALU issue, not on the LDS.
constexpr int RS32 = 132;   // fp32 rows of 128
constexpr int RS16 = 136;   // fp16 rows of 128
constexpr int RS16S = 72;   // fp16 rows of 64
constexpr int LDS_A = 0;
constexpr int LDS_B = 33792;
constexpr int LDS_BV = LDS_B + 17408;
constexpr int LDS_C = 68608;
constexpr int LDS_W = 102400;
constexpr int LDS_AQ = 119808;
constexpr int LDS_AK = 129024;
constexpr int LDS_GM = 138240;      // the gate cumsum's block middle rows 16 I + 7 [4][128] fp32 (2 KiB; 2304 bytes free)
constexpr int LDS_F = 142592;
constexpr int LDS_WT = 151808;
constexpr int LDS_BETA = 153856;
constexpr int LDS_DT = 154112;    // dt_bias of the head (gate-in-kernel) fp32 [128]
constexpr int LDS_L = 154624;     // A_kk diagonal blocks, transposed: [block][column][row], rows padded to 20
constexpr int LDS_TOTAL = 159744;
// per-channel factor rows of LDS_F
constexpr int F_A = 0;      // a_I = e^{Gamma_m(I) - Gamma_{16I-1}}, I = 1..3          (rows 0..2)
constexpr int F_B = 3;      // b_IJ = e^{Gamma_{16I-1} - Gamma_m(J)}, row 3 + I(I-1)/2 + J (rows 3..8)
constexpr int F_X = 9;      // x_I = e^{Gamma_m(I)}                                    (rows 9..12)
constexpr int F_Y = 13;     // y_I = e^{Gamma_c - Gamma_m(I)}                          (rows 13..16)
constexpr int F_DEC = 17;   // e^{Gamma_c}
constexpr int F_ROWS = 18;

constexpr uint32_t PLAN_MAGIC = 0x4b443535u;  // "KD55"
// Table: a header, then four lists.  The chain list holds every piece run by the chunk kernel (a whole sequence, the
// first piece of a split sequence from its true start state, or a later piece from S = 0 carrying its transition);
// the scan list holds the split sequences (the start states of their later pieces and their final states are composed
// after the chunk kernel); the fixup list holds one task per group of up to FX_GROUP chunks of a later piece (their
// outputs get R S_start added); the compose list holds the checkpoints inside later pieces (row = P S_start + S_local).
enum { H_MAGIC = 0, H_N, H_T, H_NCHUNK, H_EVERY, H_CKROWS, H_OFF_FINAL, H_NFINAL, H_OFF_FIX, H_NFIX, H_OFF_SCAN,
       H_NSCAN, H_NSLOTS, H_OFF_CKC, H_NCKC, H_NRSLOTS, H_NCKSLOTS, H_OFF_WG, H_WORDS = 20 };
// one piece entry: chunks [0, nch) starting at sequence chunk `first` of sequence n, tokens [t_start, t_start + len)
enum { C_SEQ = 0, C_NCH, C_TSTART, C_LEN, C_CKSINGLE, C_CKROW0, C_FIRST, C_FLAGS, C_SLOT, C_SEQCH, C_RBASE, C_CKWS,
       C_CKWS1, C_WORDS = 13 };
// C_FLAGS: PIECE_FIX: a non-first piece of a split sequence (runs from S = 0 carrying its transition, writes fp16
// partial outputs and the per-chunk correction operands R); PIECE_LAST: the entry ends an unsplit sequence (writes the
// final state); PIECE_STORE_END: the first piece of a split sequence (its end state is the second piece's start)
enum { PIECE_FIX = 1, PIECE_LAST = 2, PIECE_STORE_END = 4 };
enum { S_SEQ = 0, S_NP, S_SLOT0, S_WORDS = 4 };  // scan entry: sequence, pieces, slot of piece 0
enum { X_TSTART = 0, X_LEN, X_RSLOT, X_SSLOT, X_WORDS = 4 };  // fixup task: token rows of a chunk group, first R slot,
                                                              // start-state slot
// compose task: ck_idx position, ck slot, start slot, kind (1: the single checkpoint, 2: an every-n row); the plan
// schedules both kinds from the layout, the launch's checkpoint mode picks one
enum { K_CKIDX = 0, K_WSSLOT, K_SSLOT, K_KIND, K_WORDS = 4 };

typedef _Float16 half_t;

__device__ __forceinline__ f32x4 mfma32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma32bf(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(f16x4 a, f16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
// storage position of index q (0..31) inside a permuted 32-block: q = 16h + 4g + e  ->  8g + 4h + e
__device__ __forceinline__ int pos32(int q) { return ((q >> 2) & 3) * 8 + ((q >> 4) << 2) + (q & 3); }
__device__ __forceinline__ int pos64(int q) { return (q & 32) + pos32(q & 31); }
// Channel swizzle of the fp32 row arrays (gate / Gamma, q^ fi, k^ fi, k^ fj; 132-float rows): logical channel c is
// stored at c ^ (((c >> 5) & 3) << 2), i.e. the four 16-byte slots of the 16-channel segment of raw thread cb are
// permuted by slot ^= cb >> 1.  The eight raw threads of a row then write 16-byte slots on distinct banks (unswizzled,
// segments cb and cb + 4 sit 256 bytes apart and their writes conflict: 128 vs 55 cycles per wave instruction).
__device__ __forceinline__ int swz(int c) { return c ^ (((c >> 5) & 3) << 2); }
// hi + lo bf16 split of two fp32 values, each pair packed in one word (element 0 in the low half): hi = RNE(x),
// lo = RNE(x - hi), one v_cvt_pk_bf16_f32 per pair
__device__ __forceinline__ void split_bf16x2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
    hi = f2bf2(x0, x1);
    const float h0 = __uint_as_float(hi << 16), h1 = __uint_as_float(hi & 0xffff0000u);
    lo = f2bf2(x0 - h0, x1 - h1);
}
__device__ __forceinline__ bf16x8 as_bf16x8(const uint32_t (&w)[4]) {
    return __builtin_bit_cast(bf16x8, u32x4{w[0], w[1], w[2], w[3]});
}
// 2^x (v_exp_f32)
__device__ __forceinline__ float exp2_(float x) { return __builtin_amdgcn_exp2f(x); }
// sigmoid through the hardware reciprocal (v_rcp_f32, within 1 ulp): the IEEE division of sigmoidf_ is a sequence of
// about ten instructions, and the raw-row phase takes 17 sigmoids per thread and chunk
__device__ __forceinline__ float sigmoid_rcp(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
// A per-token log-decay below KDA355_MIN_LOG_DECAY (-9) is raised to it: the diagonal Gram blocks hold e^{+-8 g} over
// 8 tokens, inside 2^{+-104} for g >= -9, where the factors and the low halves of their bf16 pairs stay normal (the
// MFMAs flush subnormal operands; at -11 the factors reach 2^-127).  The state change this makes is below e^{-9} =
// 1.2e-4 of the affected channel's value (a decay of e^{-9} instead of a smaller one).  NaN passes through unchanged.
__device__ __forceinline__ float clamp_decay(float g) { return g < KDA355_MIN_LOG_DECAY ? KDA355_MIN_LOG_DECAY : g; }
// the same limit for a log-decay already in log2 units
constexpr float LOG2E = 1.4426950408889634f;
__device__ __forceinline__ float clamp_decay2(float g) {
    constexpr float lim = KDA355_MIN_LOG_DECAY * LOG2E;
    return g < lim ? lim : g;
}
// Gate-in-kernel constant of a head: An = -e^{A_log} log2(e), so that e^{-e^{A_log} (x + dt_bias)} =
// 2^{An x + An dt_bias} is one FMA (An dt_bias per channel sits in LDS) and one v_exp_f32
__device__ __forceinline__ float gate_an(float alog) { return -__expf(alog) * LOG2E; }
// a float read through the scalar (constant address space) cache
typedef const __attribute__((address_space(4))) float cfloat_t;

// Workgroup barrier for LDS traffic only.  __syncthreads() also fences global memory (s_waitcnt vmcnt(0)), which
// would wait for the next chunk's prefetched loads and for the output stores at every phase boundary; the waves of
// this kernel exchange data through LDS alone, so completing the LDS operations (lgkmcnt(0)) is sufficient.

// Sum over each group of 8 consecutive lanes (quad swaps, then the mirrored quad).
__device__ __forceinline__ float sum8(float x) {
    x += dpp<0xB1>(x);
    x += dpp<0x4E>(x);
    x += dpp<0x141>(x);
    return x;
}

struct PfParams {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const void* g;
    const void* beta;
    const float* A_log;
    const float* dt_bias;
    uint16_t* out;
    float* state_pool;
    const int32_t* state_idx;
    const uint8_t* has_init;
    const float* init_state;
    float* final_state;
    void* ck_pool;
    const int32_t* ck_idx;
    const int32_t* tab;
    int64_t qkv_rs, g_rs, beta_rs, out_rs;
    int64_t state_ss, state_slots, ck_ss, ck_slots;
    int N, H;
    float scale, lb;
    uint32_t flags;
    int ck_bf16;
    float* ws;   // split sequences: [3][slots][H][128][128] fp32 = local end states, transitions, start states;
                 // then [ck slots][2][H][128][128] fp32 checkpoint (local state, transition) pairs; then
                 // [R slots][H][64][128] fp16 correction operands
};

// Raw inputs of one chunk row slice: row r, channels 16 cb .. 16 cb + 15.
struct RawRow {
    u32x4 q[2], k[2], v[2];
    u32x4 g[4];  // fp32 log-decay (4 x 4 floats), or bf16 raw gate in g[0..1]
    uint32_t beta;  // fp32 bits, or the bf16 raw beta in the low half (converted when the chunk is consumed)
};

// Raw buffer descriptor over the rows [t0, t0 + L) of one token-major stream (row pitch `pitch` bytes, `bytes` bytes
// per row used): a row past the chunk end lies outside num_records, and the buffer load returns zeros for it.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void* base, int L, int64_t pitch, int bytes) {
    const int num = L > 0 ? (int)((int64_t)(L - 1) * pitch + bytes) : 0;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, num, 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t rs, int off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
}

// One chunk's raw row slice for this thread (row r, channels 16 cb .. 16 cb + 15); rows >= L read as zeros.  The
// next chunk's slice is issued in three parts in three phases (q and k; v and beta; the gate): the 80 KiB a chunk
// loads take ~1.3 k cycles of the CU's address unit, and issued at once they stall the waves that issue them.
__device__ __forceinline__ void load_row_qk(const PfParams& p, int h, int t0, int L, int r, int cb, RawRow& x) {
    const int64_t o = (int64_t)t0 * p.qkv_rs + (int64_t)h * D;
    const int64_t qp = p.qkv_rs * 2;
    const int qo = r * (int)qp + 32 * cb;
    const __amdgpu_buffer_rsrc_t rq = rows_rsrc(p.q + o, L, qp, 256);
    const __amdgpu_buffer_rsrc_t rk = rows_rsrc(p.k + o, L, qp, 256);
    x.q[0] = bload16(rq, qo); x.q[1] = bload16(rq, qo + 16);
    x.k[0] = bload16(rk, qo); x.k[1] = bload16(rk, qo + 16);
}
__device__ __forceinline__ void load_row_vb(const PfParams& p, int h, int t0, int L, int r, int cb, bool RB, RawRow& x) {
    const int64_t o = (int64_t)t0 * p.qkv_rs + (int64_t)h * D;
    const int64_t qp = p.qkv_rs * 2;
    const int qo = r * (int)qp + 32 * cb;
    const __amdgpu_buffer_rsrc_t rv = rows_rsrc(p.v + o, L, qp, 256);
    x.v[0] = bload16(rv, qo); x.v[1] = bload16(rv, qo + 16);
    const int es = RB ? 2 : 4;
    const int64_t bp = p.beta_rs * es;
    const __amdgpu_buffer_rsrc_t rb =
        rows_rsrc(reinterpret_cast<const unsigned char*>(p.beta) + ((int64_t)t0 * p.beta_rs + h) * es, L, bp, es);
    x.beta = RB ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rb, r * (int)bp, 0, 0)
                : __builtin_amdgcn_raw_buffer_load_b32(rb, r * (int)bp, 0, 0);
}
template <bool RG>
__device__ __forceinline__ void load_row_g(const PfParams& p, int h, int t0, int L, int r, int cb, RawRow& x) {
    const int64_t go = (int64_t)t0 * p.g_rs + (int64_t)h * D;
    if (RG) {
        const int64_t gp = p.g_rs * 2;
        const __amdgpu_buffer_rsrc_t rg = rows_rsrc(reinterpret_cast<const uint16_t*>(p.g) + go, L, gp, 256);
        const int off = r * (int)gp + 32 * cb;
        x.g[0] = bload16(rg, off); x.g[1] = bload16(rg, off + 16);
        x.g[2] = u32x4{0u, 0u, 0u, 0u}; x.g[3] = x.g[2];
    } else {
        const int64_t gp = p.g_rs * 4;
        const __amdgpu_buffer_rsrc_t rg = rows_rsrc(reinterpret_cast<const float*>(p.g) + go, L, gp, 512);
        const int off = r * (int)gp + 64 * cb;
        x.g[0] = bload16(rg, off); x.g[1] = bload16(rg, off + 16);
        x.g[2] = bload16(rg, off + 32); x.g[3] = bload16(rg, off + 48);
    }
}
template <bool RG>
__device__ __forceinline__ void load_row(const PfParams& p, int h, int t0, int L, int r, int cb, bool RB, RawRow& x) {
    load_row_qk(p, h, t0, L, r, cb, x);
    load_row_vb(p, h, t0, L, r, cb, RB, x);
    load_row_g<RG>(p, h, t0, L, r, cb, x);
}

__device__ __forceinline__ void unpack16(const u32x4 (&w)[2], float (&f)[16]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f[8 * i + 2 * j] = bf2f(w[i][j] & 0xffffu);
            f[8 * i + 2 * j + 1] = bf2f(w[i][j] >> 16);
        }
}

// V-major state rows of this lane: v = 16w + m, k = 16dt + 4g .. + 3
__device__ __forceinline__ void store_state(float* dst, const f32x4 (&S)[8], int w, int g, int m) {
    float* row = dst + (16 * w + m) * D + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(row + 16 * dt) = S[dt];
}
__device__ __forceinline__ void store_state_bf16(uint16_t* dst, const f32x4 (&S)[8], int w, int g, int m) {
    uint16_t* row = dst + (16 * w + m) * D + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
        u32x2 o;
        o.x = f2bf(S[dt][0]) | (f2bf(S[dt][1]) << 16);
        o.y = f2bf(S[dt][2]) | (f2bf(S[dt][3]) << 16);
        *reinterpret_cast<u32x2*>(row + 16 * dt) = o;
    }
}

// The operand of this lane tile (rows a = 16 w + m, columns b = 16 dt + 4 g + e of a [128][128] fp32 array) stored in
// the scan's blocked order: element (a, b) at ((a / 4) * 128 + b) * 4 + a % 4, i.e. for every group of 4 rows, the
// 4 values of each column contiguous and the columns in order.  A scan lane's 4 values of one column are then one
// 16-byte load and neighbouring lanes (columns) read neighbouring 16 bytes.  Staged through LDS rows of RS32 floats:
// every thread writes its tile row-major, one barrier, then every thread gathers 8 four-row column pieces.
__device__ __forceinline__ void stage_state(float* stage, const f32x4 (&S)[8], int w, int g, int m) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(stage + (16 * w + m) * RS32 + 16 * dt + 4 * g) = S[dt];
}
__device__ __forceinline__ void copy_staged_blocked(float* dst, const float* stage) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int i = threadIdx.x + PF_THREADS * j, a4 = i >> 7, b = i & 127;
        const f32x4 v = {stage[(4 * a4) * RS32 + b], stage[(4 * a4 + 1) * RS32 + b], stage[(4 * a4 + 2) * RS32 + b],
                         stage[(4 * a4 + 3) * RS32 + b]};
        *reinterpret_cast<f32x4*>(dst + 4 * i) = v;
    }
}
// A staged [128][128] fp32 array as fp16 (RNE; 16384 values) in the order: element (a, b) at
// ((a / 8) * 128 + b) * 8 + a % 8, i.e. the 8 values of each column in one group of 8 rows are 16 contiguous bytes,
// the operand of one lane of a 16x16x32 MFMA.  The transition is an fp16 MFMA operand at every chunk of the walk
// that forms it, so one more fp16 rounding here adds an error of the same kind, not a new one.
__device__ __forceinline__ void copy_staged_h(half_t* dst, const float* stage) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = threadIdx.x + PF_THREADS * j, a8 = i >> 7, b = i & 127;
        f16x8 v;
#pragma unroll
        for (int r = 0; r < 8; ++r) v[r] = (half_t)stage[(8 * a8 + r) * RS32 + b];
        *reinterpret_cast<f16x8*>(dst + 8 * i) = v;
    }
}

// One item of a chunk-kernel workgroup: a (chain entry, head) pair's table words, and for pool layouts the state row
// and the aligned word holding has_initial_state[n]; alog = A_log[h] for the gate-in-kernel form.
struct ItemWords {
    int h, n, nch, tstart, len, first, pflags, slot, seqch, ck_row0, ck_single_raw;
    const int32_t* e;  // the chain entry (the later-piece words are read where they are used)
    int64_t row;
    uint32_t hword;
    float alog;
};

// The chunk walk with outputs, checkpoints and states.  P1 = true compiles in the pieces of split sequences: an entry
// flagged PIECE_FIX starts from S = 0 and also carries its state transition P (S_end = P S_start + S_loc); its outputs
// are partial (fp16, without the S_start term), and for every chunk it stores R = Q~ P + A_qk (-W P), the operand of
// the correction O += scale R S_start; its checkpoints go to the workspace as (S_loc, P) pairs.
// PREC = true (KDA355_PF_PRECISE) carries five operands of the solve and the state update as fp16 pairs (hi = RNE(x),
// lo = RNE(x - hi): 22 bits) instead of single fp16 values: -A_IJ, T_II, the solved blocks X_J, the right-hand side
// before T_II, and V' (-W P for a transition).  On chunks of nearly parallel keys with beta ~ 1 the substitution
// cancels, and these single roundings set the state error: the reference eval's deep-layer probe measures 9.3e-4
// relative Frobenius with single operands and 4.9e-4 with the pairs; config 1 takes ~11 % longer (more MFMAs in the
// dependent chain of the solve, twice as many in the state update).
template <bool RG, bool P1, bool PREC>
__global__ void __launch_bounds__(PF_THREADS, 1)
    chunk_kernel(PfParams p, const int32_t* __restrict__ tab, const int32_t* __restrict__ ck_idx, int list_off) {
    extern __shared__ __align__(16) unsigned char lds[];
    float* sG = reinterpret_cast<float*>(lds + LDS_A);       // gate / Gamma, then k^ fi
    float* sKA = sG;
    float* sQA = reinterpret_cast<float*>(lds + LDS_B);      // q^ fi
    half_t* sQt = reinterpret_cast<half_t*>(lds + LDS_B);    // Q~ (channels permuted)
    float* sKB = reinterpret_cast<float*>(lds + LDS_C);      // k^ fj
    half_t* sKd = reinterpret_cast<half_t*>(lds + LDS_C);    // Kd^T (tokens permuted)
    half_t* sW = reinterpret_cast<half_t*>(lds + LDS_BV);    // W (channels permuted), in region B's upper half
    const uint16_t* sV = reinterpret_cast<const uint16_t*>(lds + LDS_W);  // this chunk's raw v rows (bf16)
    half_t* sAq = reinterpret_cast<half_t*>(lds + LDS_AQ);   // A_qk (columns permuted)
    half_t* sAk = reinterpret_cast<half_t*>(lds + LDS_AK);   // -A_kk off-diagonal blocks, T_II diagonal blocks
    float* sL = reinterpret_cast<float*>(lds + LDS_L);       // A_kk diagonal blocks, column-major [4][16][20]
    float* sF = reinterpret_cast<float*>(lds + LDS_F);       // per-channel factors [18][128]
    float* sWt = reinterpret_cast<float*>(lds + LDS_WT);     // segment totals of the gate cumsum [4][128]
    float* sGM = reinterpret_cast<float*>(lds + LDS_GM);     // the cumsum's block middle rows 16 I + 7 [4][128]
    float* sBeta = reinterpret_cast<float*>(lds + LDS_BETA);
    float* sDT = reinterpret_cast<float*>(lds + LDS_DT);

    const int H = p.H;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    // The workgroup's items (item = chain entry * H + head): item blockIdx.x alone, or, when the table holds workgroup
    // lists (unsplit layouts with more (chain, head) pairs than CUs), the items of list blockIdx.x in turn.  An item's
    // table words are read when the item before it starts; its first rows and gate dt_bias are fetched during the
    // last chunk of the item before it, and its start state right after that item's final state is stored, so only a
    // workgroup's first item pays the start-up of loading rows and state.
    // Uniform table reads through a __restrict__ pointer are scalar loads, which never join the vector-memory counter
    // that the prefetched rows are waited on with.
    const int32_t* wl = nullptr;
    int kpos = 0, kend = 1;
    if (!P1 && tab[H_OFF_WG] > 0) {
        wl = tab + tab[H_OFF_WG];
        kpos = wl[blockIdx.x];
        kend = wl[blockIdx.x + 1];
    }
    const bool pool = (p.flags & KDA355_PF_POOL) != 0;
    const bool RB = (p.flags & KDA355_PF_RAW_BETA) != 0;
    const bool NORM = (p.flags & KDA355_PF_NORMALIZE_QK) != 0;
    auto load_item = [&](int kp) {
        ItemWords it;
        const int item = wl ? wl[gridDim.x + 1 + kp] : (int)blockIdx.x;
        const int c = item / H;
        it.h = item - c * H;
        const int32_t* e = tab + list_off + C_WORDS * c;
        it.n = e[C_SEQ];
        it.nch = e[C_NCH];
        it.tstart = e[C_TSTART];
        it.len = e[C_LEN];
        it.first = e[C_FIRST];
        it.pflags = e[C_FLAGS];
        it.slot = e[C_SLOT];
        it.seqch = e[C_SEQCH];
        it.ck_row0 = e[C_CKROW0];
        it.ck_single_raw = e[C_CKSINGLE];
        it.e = e;
        it.row = -1;
        it.hword = 0;
        if (pool) {
            // the pool row and has_initial_state[n] in one round: the flag by a scalar read of its aligned word through
            // the constant address space (read-only for the kernel; a uniform address there becomes s_load_dword, so
            // no vector load has to be waited for).  The aligned word may cover bytes next to the flag but never
            // leaves the flag's page.
            typedef const __attribute__((address_space(4))) uint32_t cword_t;
            typedef const __attribute__((address_space(4))) int32_t cint_t;
            it.row = *reinterpret_cast<cint_t*>(reinterpret_cast<uintptr_t>(p.state_idx + it.n));
            it.hword = *reinterpret_cast<cword_t*>(reinterpret_cast<uintptr_t>(p.has_init + it.n) & ~(uintptr_t)3);
        }
        it.alog = RG ? *reinterpret_cast<cfloat_t*>(reinterpret_cast<uintptr_t>(p.A_log + it.h)) : 0.f;
        return it;
    };
    // the start state's source: none for a later piece (it runs from zero) and for a pool sequence without an initial
    // state; S is loaded through a descriptor of no records when there is none
    auto state_source = [&](const ItemWords& it) -> const float* {
        if (P1 && (it.pflags & PIECE_FIX)) return nullptr;
        if (pool) {
            const uintptr_t ha = reinterpret_cast<uintptr_t>(p.has_init + it.n);
            const bool hinit = ((it.hword >> (8 * (ha & 3))) & 0xffu) != 0;
            return (it.row >= 0 && it.row < p.state_slots && hinit)
                       ? p.state_pool + it.row * p.state_ss + (int64_t)it.h * D * D : nullptr;
        }
        return p.init_state ? p.init_state + ((int64_t)it.n * H + it.h) * D * D : nullptr;
    };
    const int every = tab[H_EVERY];
    const int64_t ws_arr = (int64_t)tab[H_NSLOTS] * H * D * D;  // floats per workspace array
    const int64_t ck_words = (int64_t)tab[H_NCKSLOTS];
    float* ws_ck = p.ws + 3 * ws_arr;                            // checkpoint (S_loc, P) pairs
    half_t* ws_r = reinterpret_cast<half_t*>(ws_ck + ck_words * 2 * H * D * D);  // R operands

    // ---- prologue.  Loads are issued in the order they are needed and none sits under a branch (the memory counter
    // completes in issue order, and a load on one path only makes the compiler wait for everything older): the first
    // chunk's rows (P0), the gate's dt_bias (P0), then the initial state, first used by the first walk.
    int tid = threadIdx.x, lane = tid & 63, m = lane & 15, g = lane >> 4, r = tid >> 3, cb = tid & 7;
    // The prologue's memory reads are issued in two dependent rounds: first what depends on the launch alone (the
    // table header, the chain entry, the gate's dt_bias, which is therefore waited for without waiting for the rows),
    // then what depends on the chain entry (the first chunk's rows, the pool row and its has_initial_state flag); the
    // initial state is issued last and only waited for before the first walk.  Every table word the loop uses is read
    // here (empty asm operands pin the reads in the first round), so the first LDS barrier has no scalar read left to
    // wait for.
    ItemWords cur = load_item(kpos);
    float dtb = RG ? p.dt_bias[cur.h * D + (tid & (D - 1))] : 0.f;
    asm volatile("" ::"s"(every), "s"(ws_arr), "s"(cur.ck_row0), "s"(cur.ck_single_raw), "s"(ck_words), "s"(cur.alog),
                 "s"(p.ws));
    RawRow nx;
    // an empty sequence loads nothing
    load_row<RG>(p, cur.h, cur.tstart, cur.nch > 0 ? min(64, cur.len) : 0, r, cb, RB, nx);
    f32x4 S[8];
    // initial state (lane: v = 16w + m, k = 16dt + 4g + e)
    auto load_start_state = [&](const float* src) {
        // base and size taken through readfirstlane: a descriptor the compiler cannot see as wave-uniform becomes a
        // waterfall loop
        const int nrec = __builtin_amdgcn_readfirstlane(src ? D * D * 4 : 0);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            uniform_ptr(src ? static_cast<const void*>(src) : static_cast<const void*>(p.q)), (short)0, nrec, 0x00020000);
        const int voff = ((16 * w + (threadIdx.x & 15)) * D + 4 * ((threadIdx.x >> 4) & 3)) * 4;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
            S[dt] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 64 * dt, 0, 0));
    };
    load_start_state(state_source(cur));

    const int ck_mode = (p.flags & KDA355_PF_CK_EVERY) ? 2 : ((p.flags & KDA355_PF_CK_SINGLE) ? 1 : 0);
    // gate-in-kernel constants for this thread's 16 channels
    float An = 0.f;
    if (RG) {
        An = gate_an(cur.alog);
        if (tid < D) sDT[tid] = An * dtb;
    }
    // A_qk blocks (0,1) and (2,3) are read by the walk and never written by the Gram phase
    for (int e = tid; e < 2 * 16 * 16; e += PF_THREADS) {
        const int b = e >> 8, ii = (e >> 4) & 15, jj = e & 15;
        sAq[(32 * b + ii) * RS16S + 32 * b + pos32(16 + jj)] = (half_t)0.f;
    }
    lds_barrier();  // sDT and the zeroed A_qk blocks are visible to every wave

    for (;;) {  // the workgroup's items
        const int h = cur.h, n = cur.n, nch = cur.nch, tstart = cur.tstart, len = cur.len, first = cur.first;
        const int pflags = cur.pflags, slot = cur.slot, seqch = cur.seqch;
        const bool fix = P1 && (pflags & PIECE_FIX);
        float* ws_h = p.ws + ((int64_t)slot * H + h) * D * D;        // this piece-head in array 0 (+ ws_arr: 1, 2)
        const int ck_row0 = cur.ck_row0;
        const int ck_single = (ck_mode == 1) ? cur.ck_single_raw : 0;
        // the next item's head, first token, length and chunk count, for the rows fetched during this item's last
        // chunk; its other words are read when it starts
        const bool more = kpos + 1 < kend;
        int nx_h = 0, nx_t = 0, nx_len = 0, nx_nch = 0;
        float dtb_next = 0.f;
        if (more) {
            const int it2 = wl[gridDim.x + 2 + kpos], c2 = it2 / H;
            const int32_t* e2 = tab + list_off + C_WORDS * c2;
            nx_h = it2 - c2 * H;
            nx_nch = e2[C_NCH];
            nx_t = e2[C_TSTART];
            nx_len = e2[C_LEN];
            if (RG)  // An dt_bias of the next item's head (its sDT contents)
                dtb_next = gate_an(*reinterpret_cast<cfloat_t*>(reinterpret_cast<uintptr_t>(p.A_log + nx_h))) *
                           p.dt_bias[nx_h * D + (threadIdx.x & (D - 1))];
        }
        f32x4 Pm[8];  // fix: the transition, P[k][k'] at (k = 16dt + 4g + e, k' = 16w + m); starts as the identity
        if (fix) {
#pragma unroll
            for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                for (int e = 0; e < 4; ++e) Pm[dt][e] = (16 * dt + 4 * g + e == 16 * w + m) ? 1.f : 0.f;
        }
        auto ck_store = [&](int64_t rr) {
            if (rr < 0 || rr >= p.ck_slots) return;
            if (p.ck_bf16)
                store_state_bf16(reinterpret_cast<uint16_t*>(p.ck_pool) + rr * p.ck_ss + (int64_t)h * D * D, S, w, g, m);
            else
                store_state(reinterpret_cast<float*>(p.ck_pool) + rr * p.ck_ss + (int64_t)h * D * D, S, w, g, m);
        };

        for (int cl = 0; cl < nch; ++cl) {
            // Lane indices are re-derived every chunk from an opaque copy so that the per-lane LDS addresses of all
            // phases are recomputed where they are used instead of being kept live (and spilled) across the whole loop.
            tid = threadIdx.x;
            asm volatile("" : "+v"(tid));
            lane = tid & 63;
            m = lane & 15;
            g = lane >> 4;
            r = tid >> 3;
            cb = tid & 7;
            const int t0 = tstart + 64 * cl, L = min(64, len - 64 * cl);
            // the rows fetched during this chunk: the next chunk's, or during an item's last chunk the next item's
            // first
            const bool pf_here = cl + 1 < nch, pf = pf_here || more;
            const int pf_h = pf_here ? h : nx_h, pf_t = pf_here ? t0 + 64 : nx_t;
            const int pf_L = pf_here ? min(64, len - 64 * (cl + 1)) : (nx_nch > 0 ? min(64, nx_len) : 0);
            // ================= P0: this chunk's raw rows (prefetched during the previous chunk)
            // The raw q and k stay in registers until P2 (the next chunk's q, k loads reuse them from P5 on); the raw v
            // goes to an LDS slot that only this thread reads back (the W area, which is free until P6), so its
            // registers die here and the next chunk's v loads reuse them without a loop-carried copy.
            *reinterpret_cast<u32x4*>(lds + LDS_W + r * (2 * RS16) + 32 * cb) = nx.v[0];
            *reinterpret_cast<u32x4*>(lds + LDS_W + r * (2 * RS16) + 32 * cb + 16) = nx.v[1];
            float gv[16];
            if (RG) {
                float rg[16];
                const u32x4 gg[2] = {nx.g[0], nx.g[1]};
                unpack16(gg, rg);
                // g log2(e) = lb log2(e) sigmoid(e^{A_log} (x + dt_bias)), the sigmoid as 1 / (1 + 2^{An x + An dt})
                // (one FMA, v_exp_f32, one add, v_rcp_f32), already in the log2 units of the cumsum.  Every row is
                // computed; rows >= L get a zero multiplier (their raw gate reads as 0, so the sigmoid is finite): a
                // computation under the row mask would branch per value and wait for every outstanding LDS read.
                const float lbm = (r < L) ? p.lb * LOG2E : 0.f;
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const f32x4 adt4 = *reinterpret_cast<const f32x4*>(&sDT[16 * cb + 4 * q4]);  // An dt_bias
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        gv[4 * q4 + e] = clamp_decay2(
                            lbm * __builtin_amdgcn_rcpf(1.0f + exp2_(fmaf(An, rg[4 * q4 + e], adt4[e]))));
                }
            } else {  // natural-log units here; the cumsum scales them by log2(e) as it adds
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) gv[4 * i + j] = clamp_decay(__uint_as_float(nx.g[i][j]));
            }
            const float bx = RB ? sigmoid_rcp(bf2f(nx.beta)) : __uint_as_float(nx.beta);
            const float bt = (r >= L) ? 0.f : bx;
            float rq = 1.f, rk = 1.f;
            if (NORM) {  // F.normalize(x, eps=1e-6) = x / max(|x|, 1e-6)  (kda/mi350x/reference.py:59-60)
                // sums of squares straight from the packed bf16 pairs (v_dot2c_f32_bf16: the products are exact in
                // fp32), so this phase unpacks no q / k value
                float sq = 0.f, sk = 0.f;
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        // element copies first: a bit cast of the vector element itself loses its index in this
                        // compiler (every j read element 0)
                        const uint32_t wq = nx.q[i][j], wk = nx.k[i][j];
                        const bf16x2_t qp = __builtin_bit_cast(bf16x2_t, wq);
                        const bf16x2_t kp = __builtin_bit_cast(bf16x2_t, wk);
                        sq = __builtin_amdgcn_fdot2_f32_bf16(qp, qp, sq, false);
                        sk = __builtin_amdgcn_fdot2_f32_bf16(kp, kp, sk, false);
                    }
                sq = sum8(sq);
                sk = sum8(sk);
                // 1 / max(|x|, 1e-6) = rsqrt(max(|x|^2, 1e-12)) through v_rsq_f32 (the IEEE sqrt is a sequence)
                rq = __builtin_amdgcn_rsqf(fmaxf(sq, 1e-12f));
                rk = __builtin_amdgcn_rsqf(fmaxf(sk, 1e-12f));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<f32x4*>(&sG[r * RS32 + 16 * cb + 4 * (i ^ (cb >> 1))]) =
                    f32x4{gv[4 * i], gv[4 * i + 1], gv[4 * i + 2], gv[4 * i + 3]};
            if (cb == 0) sBeta[r] = bt;
            lds_barrier();
            // ================= P1: gate cumsum inside 16-row segments
            {
                const int c = tid & 127, s = tid >> 7;
                float x[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) x[i] = sG[(16 * s + i) * RS32 + swz(c)];
                if (RG) {  // already in log2 units
#pragma unroll
                    for (int i = 1; i < 16; ++i) x[i] += x[i - 1];
                } else {  // natural log: the log2(e) scale goes into the adds
                    x[0] *= LOG2E;
#pragma unroll
                    for (int i = 1; i < 16; ++i) x[i] = fmaf(x[i], LOG2E, x[i - 1]);
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) sG[(16 * s + i) * RS32 + swz(c)] = x[i];
                sWt[s * 128 + c] = x[15];
                sGM[s * 128 + c] = x[7];  // the factors' reference row of block s, kept apart so P2 can overwrite sG
            }
            lds_barrier();
            // ================= P2: element factors (raw threads) and block factors (channel threads).  The block
            // middle rows and segment totals come from sGM / sWt, so each raw thread reads only its own gate row from
            // sG and can overwrite that row with k^ fi in place (no other thread reads it in this phase).
            {
                float qf[16], kf[16];
                {
                    const u32x4 a[2] = {nx.q[0], nx.q[1]}, b[2] = {nx.k[0], nx.k[1]};
                    unpack16(a, qf);
                    unpack16(b, kf);
                }
                if (NORM) {  // uniform: calls without in-kernel normalization skip the 32 multiplies by 1
#pragma unroll
                    for (int c = 0; c < 16; ++c) { kf[c] *= rk; qf[c] *= rq; }
                }
                const int I = r >> 4;
                // block i of the row: its gate values are read before its k^ fi overwrites them (one thread, in order)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int o = r * RS32 + 16 * cb + 4 * (i ^ (cb >> 1));
                    const f32x4 a = *reinterpret_cast<const f32x4*>(&sG[o]);
                    const f32x4 b = *reinterpret_cast<const f32x4*>(&sGM[I * 128 + 16 * cb + 4 * i]);
                    f32x4 kfi, kfj, qfi;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int c = 4 * i + j;
                        const float d = a[j] - b[j];  // Gamma_r - Gamma_m (the segment offset cancels)
                        const float fi = exp2_(d), fj = exp2_(-d);
                        kfi[j] = kf[c] * fi;
                        kfj[j] = kf[c] * fj;
                        qfi[j] = qf[c] * fi;
                    }
                    *reinterpret_cast<f32x4*>(&sQA[o]) = qfi;
                    *reinterpret_cast<f32x4*>(&sKB[o]) = kfj;
                    *reinterpret_cast<f32x4*>(&sKA[o]) = kfi;
                }
            }
            {
                // qd is wave-uniform (128 threads per value): the row selection below branches on the scalar unit
                const int c = tid & 127, qd = __builtin_amdgcn_readfirstlane(tid >> 7);
                const float o1 = sWt[c], o2 = o1 + sWt[128 + c], o3 = o2 + sWt[256 + c];
                // Gamma at rows 8 i + 7: block middles (sGM) and segment ends (sWt), plus the earlier segments
                float gr[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float off = (i < 2) ? 0.f : (i < 4) ? o1 : (i < 6) ? o2 : o3;
                    gr[i] = ((i & 1) ? sWt[(i >> 1) * 128 + c] : sGM[(i >> 1) * 128 + c]) + off;
                }
#pragma unroll
                for (int f = 0; f < F_ROWS; ++f) {  // unrolled: gr[] is indexed by constants only (stays in registers)
                    if ((f & 3) != qd) continue;
                    float x;
                    if (f < F_B) {                       // a_I, I = f + 1: Gamma_m(I) - Gamma_{16I-1}
                        const int I = f + 1;
                        x = gr[2 * I] - gr[2 * I - 1];
                    } else if (f < F_X) {                // b_IJ
                        const int t = f - F_B;
                        const int I = t < 1 ? 1 : (t < 3 ? 2 : 3);
                        const int J = t - (I * (I - 1)) / 2;
                        x = gr[2 * I - 1] - gr[2 * J];
                    } else if (f < F_Y) {
                        x = gr[2 * (f - F_X)];
                    } else if (f < F_DEC) {
                        x = gr[7] - gr[2 * (f - F_Y)];
                    } else {
                        x = gr[7];
                    }
                    sF[f * 128 + c] = exp2_(x);
                }
            }
            lds_barrier();
            // ================= P4: Gram tiles
            if (w < 4) {
                const int I = w, i = 16 * I + m;
                f32x4 akk = {0.f, 0.f, 0.f, 0.f}, aqk = akk;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const int c0 = 32 * s + 8 * g;
                    uint32_t kah[4], kal[4], qah[4], qal[4], kbh[4], kbl[4];  // bf16x8 fragments as 4 packed pairs
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf) {
                        const f32x4 ka = *reinterpret_cast<const f32x4*>(&sKA[i * RS32 + swz(c0 + 4 * hf)]);
                        const f32x4 qa = *reinterpret_cast<const f32x4*>(&sQA[i * RS32 + swz(c0 + 4 * hf)]);
                        const f32x4 kb = *reinterpret_cast<const f32x4*>(&sKB[i * RS32 + swz(c0 + 4 * hf)]);
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            const int e = 2 * hf + j;
                            split_bf16x2(ka[2 * j], ka[2 * j + 1], kah[e], kal[e]);
                            split_bf16x2(qa[2 * j], qa[2 * j + 1], qah[e], qal[e]);
                            split_bf16x2(kb[2 * j], kb[2 * j + 1], kbh[e], kbl[e]);
                        }
                    }
                    const bf16x8 Kah = as_bf16x8(kah), Kal = as_bf16x8(kal), Qah = as_bf16x8(qah), Qal = as_bf16x8(qal);
                    const bf16x8 Kbh = as_bf16x8(kbh), Kbl = as_bf16x8(kbl);
                    akk = mfma32bf(Kah, Kbh, akk);
                    akk = mfma32bf(Kah, Kbl, akk);
                    akk = mfma32bf(Kal, Kbh, akk);
                    // transposed: lane (g, m) holds row 16 I + m, columns 16 I + 4 g .. + 3
                    aqk = mfma32bf(Kbh, Qah, aqk);
                    aqk = mfma32bf(Kbl, Qah, aqk);
                    aqk = mfma32bf(Kbh, Qal, aqk);
                }
                f32x4 lt;
                f16x4 aq;
                // beta of rows 16 I + 4 g .. + 3, read whatever the mask (a read under the mask would branch and wait
                // for every outstanding LDS operation)
                const f32x4 bt4 = *reinterpret_cast<const f32x4*>(&sBeta[16 * I + 4 * g]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int rr = 4 * g + e;
                    lt[e] = (m < rr) ? bt4[e] * akk[e] : 0.f;
                    aq[e] = (half_t)((rr <= m) ? aqk[e] : 0.f);  // A_qk[16 I + m][16 I + rr], causal within the block
                }
                *reinterpret_cast<f16x4*>(&sAq[i * RS16S + pos64(16 * I + 4 * g)]) = aq;
                *reinterpret_cast<f32x4*>(&sL[(I * 16 + m) * 20 + 4 * g]) = lt;
                // T_II = (I + L_II)^-1 of this wave's block while waves 4..7 still work on the off-diagonal blocks:
                // lane j (every group of 16 lanes computes the same columns; lanes 0..15 write) solves column j by
                // right-looking substitution.  The wave reads back the block it has just written: a wave's LDS
                // operations complete in order.
                {
                    const float* Lb = sL + I * 16 * 20;  // column k of L_II is the contiguous row k
                    float x[16];
#pragma unroll
                    for (int ii = 0; ii < 16; ++ii) x[ii] = (ii == m) ? 1.f : 0.f;
#pragma unroll
                    for (int k = 0; k < 15; ++k) {  // x[k] is final: push it into the rows below
                        float col[16];
#pragma unroll
                        for (int q4 = 0; q4 < 4; ++q4) {
                            const f32x4 c4 = *reinterpret_cast<const f32x4*>(&Lb[k * 20 + 4 * q4]);
                            col[4 * q4] = c4[0]; col[4 * q4 + 1] = c4[1]; col[4 * q4 + 2] = c4[2]; col[4 * q4 + 3] = c4[3];
                        }
#pragma unroll
                        for (int ii = k + 1; ii < 16; ++ii) x[ii] -= col[ii] * x[k];
                    }
                    if (g == 0) {
#pragma unroll
                        for (int ii = 0; ii < 16; ++ii) {
                            const half_t hi = (half_t)x[ii];
                            sAk[(16 * I + ii) * RS16S + 16 * I + m] = hi;
                            // PREC: the low part in the A_qk block (I / 2, 2 + I % 2), a block of rows 0..31 and
                            // columns 32..63 that the walk never reads and the Gram phase never writes
                            if (PREC)
                                sAq[(16 * (I >> 1) + ii) * RS16S + 32 + 16 * (I & 1) + m] = (half_t)(x[ii] - (float)hi);
                        }
                    }
                }
            } else {
                const int I = (w == 4) ? 1 : ((w == 5) ? 2 : 3);
                const int J0 = (w == 7) ? 2 : 0;
                const int nJ = (w == 4 || w == 7) ? 1 : 2;
                const int i = 16 * I + m;
                f32x4 akk[2], aqk[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) { akk[t] = f32x4{0.f, 0.f, 0.f, 0.f}; aqk[t] = akk[t]; }
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const int c0 = 32 * s + 8 * g;
                    f16x8 ka, qa;
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf) {
                        const f32x4 a = *reinterpret_cast<const f32x4*>(&sKA[i * RS32 + swz(c0 + 4 * hf)]);
                        const f32x4 q4 = *reinterpret_cast<const f32x4*>(&sQA[i * RS32 + swz(c0 + 4 * hf)]);
                        const f32x4 fa = *reinterpret_cast<const f32x4*>(&sF[(F_A + I - 1) * 128 + c0 + 4 * hf]);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            ka[4 * hf + j] = (half_t)(a[j] * fa[j]);
                            qa[4 * hf + j] = (half_t)(q4[j] * fa[j]);
                        }
                    }
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        if (t < nJ) {
                            const int J = J0 + t, jr = 16 * J + m;
                            const int fb = F_B + (I * (I - 1)) / 2 + J;
                            f16x8 kb;
#pragma unroll
                            for (int hf = 0; hf < 2; ++hf) {
                                const f32x4 b = *reinterpret_cast<const f32x4*>(&sKB[jr * RS32 + swz(c0 + 4 * hf)]);
                                const f32x4 fbv = *reinterpret_cast<const f32x4*>(&sF[fb * 128 + c0 + 4 * hf]);
#pragma unroll
                                for (int j = 0; j < 4; ++j) kb[4 * hf + j] = (half_t)(b[j] * fbv[j]);
                            }
                            akk[t] = mfma32(kb, ka, akk[t]);  // transposed tiles: lane (g, m) holds row 16 I + m,
                            aqk[t] = mfma32(kb, qa, aqk[t]);  // columns 16 J + 4 g .. + 3
                        }
                    }
                }
                const float nb = -sBeta[i];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    if (t < nJ) {
                        const int J = J0 + t;
                        f16x4 ak, al, aq;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float x = nb * akk[t][e];
                            ak[e] = (half_t)x;
                            al[e] = (half_t)(x - (float)ak[e]);
                            aq[e] = (half_t)aqk[t][e];
                        }
                        *reinterpret_cast<f16x4*>(&sAk[i * RS16S + 16 * J + 4 * g]) = ak;
                        // PREC: the low part goes to the unused mirrored block (J, I) of the same array
                        if (PREC) *reinterpret_cast<f16x4*>(&sAk[(16 * J + m) * RS16S + 16 * I + 4 * g]) = al;
                        *reinterpret_cast<f16x4*>(&sAq[i * RS16S + pos64(16 * J + 4 * g)]) = aq;
                    }
                }
            }
            // no barrier here: the reads below touch only the raw v staging and the thread's own q^ fi / k^ fj rows,
            // which the Gram phase neither writes nor overwrites; the barrier before the layouts orders every Gram read
            // of regions B and C before they are rewritten
            // ================= P5: Q~, Kd^T, beta v into their walk layouts (raw threads)
            // The initial state loads (issued in the prologue or at the item's start) complete here, before any
            // next-chunk row is in flight: an empty use of S makes the compiler's wait for them fall at this point,
            // where in every later chunk only the long-finished output stores are outstanding, instead of before each
            // walk, where it would also wait for the prefetched rows.
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) asm volatile("" : "+v"(S[dt]));
            // the next chunk's q, k rows: issued here, consumed at the next P0 (their registers are free during P1..P4)
            if (pf) load_row_qk(p, pf_h, pf_t, pf_L, r, cb, nx);
            float qfi[16], kfj[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f32x4 a = *reinterpret_cast<const f32x4*>(&sQA[r * RS32 + 16 * cb + 4 * (i ^ (cb >> 1))]);
                const f32x4 b = *reinterpret_cast<const f32x4*>(&sKB[r * RS32 + 16 * cb + 4 * (i ^ (cb >> 1))]);
#pragma unroll
                for (int j = 0; j < 4; ++j) { qfi[4 * i + j] = a[j]; kfj[4 * i + j] = b[j]; }
            }
            lds_barrier();  // regions B and C are rewritten below
            {
                const int I = r >> 4;
                const int hb = cb & 1, blk = cb >> 1;
#pragma unroll
                for (int gq = 0; gq < 4; ++gq) {
                    const f32x4 xf = *reinterpret_cast<const f32x4*>(&sF[(F_X + I) * 128 + 16 * cb + 4 * gq]);
                    f16x4 o;
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[e] = (half_t)(qfi[4 * gq + e] * xf[e]);
                    *reinterpret_cast<f16x4*>(&sQt[r * RS16 + 32 * blk + 8 * gq + 4 * hb]) = o;
                }
                // Kd^T row of key channel k is stored at row 16 (k / 16) + (k % 16 ^ k / 16): the 8 channel blocks of a
                // column write then land on 8 different banks
                const int pr = pos64(r);
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float y = sF[(F_Y + I) * 128 + 16 * cb + e];
                    sKd[(16 * cb + (e ^ cb)) * RS16S + pr] = (half_t)(kfj[e] * y);
                }
            }
            // no barrier here: the solve reads k^ fi (region A), the raw v rows, -A_kk / T_II, the factors and beta,
            // none of which the layouts above write; it writes W into region B's upper half, whose last reader (the
            // operand reads before the layouts) passed the barrier above.  The walk reads the layouts after the solve's
            // barrier.
            // ================= P6: W and U by block forward substitution (wave w: channel / value tile w)
            if (pf) load_row_vb(p, pf_h, pf_t, pf_L, r, cb, RB, nx);
            f32x4 Ur[4];
            {
                const int c = 16 * w + m;
                f32x4 Xw[4];
                // PREC: -A_IJ, T_II, the solved blocks X_J and the right-hand side before T_II as fp16 pairs
                f16x4 Xh[4], Xl[4], Uh[4], Ul[4];
                auto split4 = [](const f32x4& x, f16x4& hi, f16x4& lo) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) { hi[e] = (half_t)x[e]; lo[e] = (half_t)(x[e] - (float)hi[e]); }
                };
#pragma unroll
                for (int I = 0; I < 4; ++I) {
                    const float xI = sF[(F_X + I) * 128 + c];
                    const f32x4 b4 = *reinterpret_cast<const f32x4*>(&sBeta[16 * I + 4 * g]);  // beta of the 4 rows
                    f32x4 aw, au;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int rw = 16 * I + 4 * g + e;
                        aw[e] = b4[e] * sKA[rw * RS32 + swz(c)] * xI;
                        au[e] = b4[e] * bf2f(sV[rw * RS16 + c]);  // beta v straight from the raw v row
                    }
#pragma unroll
                    for (int J = 0; J < I; ++J) {
                        const f16x4 A = *reinterpret_cast<const f16x4*>(&sAk[(16 * I + m) * RS16S + 16 * J + 4 * g]);
                        const f16x4 Al =
                            PREC ? *reinterpret_cast<const f16x4*>(&sAk[(16 * J + m) * RS16S + 16 * I + 4 * g]) : f16x4{};
                        aw = mfma16(A, Xh[J], aw);
                        au = mfma16(A, Uh[J], au);
                        if (PREC) {
                            aw = mfma16(A, Xl[J], aw);
                            au = mfma16(A, Ul[J], au);
                            aw = mfma16(Al, Xh[J], aw);
                            au = mfma16(Al, Uh[J], au);
                        }
                    }
                    const f16x4 T = *reinterpret_cast<const f16x4*>(&sAk[(16 * I + m) * RS16S + 16 * I + 4 * g]);
                    f16x4 bwh, bwl, buh, bul;
                    split4(aw, bwh, bwl);
                    split4(au, buh, bul);
                    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                    Xw[I] = mfma16(T, bwh, z);
                    Ur[I] = mfma16(T, buh, z);
                    if (PREC) {
                        const int tl = (16 * (I >> 1) + m) * RS16S + 32 + 16 * (I & 1) + 4 * g;
                        const f16x4 Tl = *reinterpret_cast<const f16x4*>(&sAq[tl]);
                        Xw[I] = mfma16(Tl, bwh, mfma16(T, bwl, Xw[I]));
                        Ur[I] = mfma16(Tl, buh, mfma16(T, bul, Ur[I]));
                    }
                    if (I < 3) {
                        split4(Xw[I], Xh[I], Xl[I]);
                        split4(Ur[I], Uh[I], Ul[I]);
                    }
                }
                const int pc = 32 * (c >> 5) + pos32(c & 31);
#pragma unroll
                for (int I = 0; I < 4; ++I)
#pragma unroll
                    for (int e = 0; e < 4; ++e) sW[(16 * I + 4 * g + e) * RS16 + pc] = (half_t)Xw[I][e];
            }
            // the next item's gate dt_bias for its first raw-row phase (this chunk's has read sDT; the barrier below
            // publishes the new values)
            if (RG && !pf_here && more && tid < D) sDT[tid] = dtb_next;
            lds_barrier();
            // ================= P7: the walk
            if (pf) load_row_g<RG>(p, pf_h, pf_t, pf_L, r, cb, nx);
            // every-n row 0 is the state before the sequence's first token: stored before the first walk changes S
            // (here rather than in the prologue, so that nothing before the first walk waits for the state loads)
            if (cl == 0 && ck_mode == 2 && every > 0 && first == 0) ck_store(ck_idx[ck_row0]);
            if (fix) {  // S <- (diag(d) - Kd^T W) S + Kd^T U and P <- (diag(d) - Kd^T W) P, sharing every A fragment
                f16x8 SB[4], PB[4];
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        SB[s][e] = (half_t)S[2 * s][e];
                        SB[s][4 + e] = (half_t)S[2 * s + 1][e];
                        PB[s][e] = (half_t)Pm[2 * s][e];
                        PB[s][4 + e] = (half_t)Pm[2 * s + 1][e];
                    }
                f32x4 Vp[4], Wp[4];  // W S and W P, K step outermost (eight independent MFMA chains per step)
#pragma unroll
                for (int it = 0; it < 4; ++it) { Vp[it] = f32x4{0.f, 0.f, 0.f, 0.f}; Wp[it] = Vp[it]; }
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int it = 0; it < 4; ++it) {
                        const f16x8 A = *reinterpret_cast<const f16x8*>(&sW[(16 * it + m) * RS16 + 32 * s + 8 * g]);
                        Vp[it] = mfma32(A, SB[s], Vp[it]);
                        Wp[it] = mfma32(A, PB[s], Wp[it]);
                    }
#pragma unroll
                for (int it = 0; it < 4; ++it)
#pragma unroll
                    for (int e = 0; e < 4; ++e) { Vp[it][e] = Ur[it][e] - Vp[it][e]; Wp[it][e] = -Wp[it][e]; }
                f16x8 VB[2], WB[2], VL[2], WL[2];  // V' and -W P; PREC: also their low parts (fp16 pairs)
#pragma unroll
                for (int s = 0; s < 2; ++s)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        VB[s][e] = (half_t)Vp[2 * s][e];
                        VB[s][4 + e] = (half_t)Vp[2 * s + 1][e];
                        WB[s][e] = (half_t)Wp[2 * s][e];
                        WB[s][4 + e] = (half_t)Wp[2 * s + 1][e];
                        VL[s][e] = (half_t)(Vp[2 * s][e] - (float)VB[s][e]);
                        VL[s][4 + e] = (half_t)(Vp[2 * s + 1][e] - (float)VB[s][4 + e]);
                        WL[s][e] = (half_t)(Wp[2 * s][e] - (float)WB[s][e]);
                        WL[s][4 + e] = (half_t)(Wp[2 * s + 1][e] - (float)WB[s][4 + e]);
                    }
                // partial O^T = S^T Q~^T + V'^T A_qk^T (fp16, to `out`) and R^T = P^T Q~^T + W'^T A_qk^T (to the
                // workspace), transposed tiles sharing the Q~ and A_qk fragments: lane (g, m) holds token 16 it + m,
                // columns 16 w + 4 g .. + 3
                half_t* rdst = ws_r + ((int64_t)(cur.e[C_RBASE] + cl) * H + h) * (64 * D) + 16 * w + 4 * g;
#pragma unroll
                for (int it = 0; it < 4; ++it) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f}, acr = acc;
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const f16x8 B = *reinterpret_cast<const f16x8*>(&sQt[(16 * it + m) * RS16 + 32 * s + 8 * g]);
                        acc = mfma32(SB[s], B, acc);
                        acr = mfma32(PB[s], B, acr);
                    }
#pragma unroll
                    for (int s = 0; s < 2; ++s)
                        if (s <= (it >> 1)) {
                            const f16x8 B = *reinterpret_cast<const f16x8*>(&sAq[(16 * it + m) * RS16S + 32 * s + 8 * g]);
                            acc = mfma32(VB[s], B, acc);
                            acr = mfma32(WB[s], B, acr);
                        }
                    f16x4 o, rr;
#pragma unroll
                    for (int e = 0; e < 4; ++e) { o[e] = (half_t)(p.scale * acc[e]); rr[e] = (half_t)acr[e]; }
                    if (16 * it + m < L)
                        *reinterpret_cast<f16x4*>(p.out + ((int64_t)t0 + 16 * it + m) * p.out_rs + (int64_t)h * D + 16 * w +
                                                  4 * g) = o;
                    *reinterpret_cast<f16x4*>(rdst + (16 * it + m) * D) = rr;
                }
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) {
                    const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sF[F_DEC * 128 + 16 * dt + 4 * g]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) { S[dt][e] *= d4[e]; Pm[dt][e] *= d4[e]; }
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        const f16x8 A = *reinterpret_cast<const f16x8*>(&sKd[(16 * dt + (m ^ dt)) * RS16S + 32 * s + 8 * g]);
                        S[dt] = mfma32(A, VB[s], S[dt]);
                        Pm[dt] = mfma32(A, WB[s], Pm[dt]);
                        if (PREC) {
                            S[dt] = mfma32(A, VL[s], S[dt]);
                            Pm[dt] = mfma32(A, WL[s], Pm[dt]);
                        }
                    }
                }
            } else {
                f16x8 SB[4];
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        SB[s][e] = (half_t)S[2 * s][e];
                        SB[s][4 + e] = (half_t)S[2 * s + 1][e];
                    }
                f32x4 Vp[4];
                // W S with the K step outermost: the four token tiles' MFMAs of one step are independent, so none
                // waits for the previous one's accumulator
#pragma unroll
                for (int it = 0; it < 4; ++it) Vp[it] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int it = 0; it < 4; ++it)
                        Vp[it] = mfma32(*reinterpret_cast<const f16x8*>(&sW[(16 * it + m) * RS16 + 32 * s + 8 * g]), SB[s],
                                        Vp[it]);
#pragma unroll
                for (int it = 0; it < 4; ++it)
#pragma unroll
                    for (int e = 0; e < 4; ++e) Vp[it][e] = Ur[it][e] - Vp[it][e];
                f16x8 VB[2], VL[2];  // V'; PREC: also its low part (an fp16 pair)
#pragma unroll
                for (int s = 0; s < 2; ++s)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        VB[s][e] = (half_t)Vp[2 * s][e];
                        VB[s][4 + e] = (half_t)Vp[2 * s + 1][e];
                        VL[s][e] = (half_t)(Vp[2 * s][e] - (float)VB[s][e]);
                        VL[s][4 + e] = (half_t)(Vp[2 * s + 1][e] - (float)VB[s][4 + e]);
                    }
                // O^T = S^T Q~^T + V'^T A_qk^T: the same fragments with the MFMA operands swapped give the transposed
                // tile, so lane (g, m) holds token 16 it + m, values 16 w + 4 g .. + 3 and stores them to `out` with
                // one 8-byte store (the 8 waves' 32-byte pieces of a token row meet in the L2)
                {
                    f32x4 ao[4];  // K step outermost here too
#pragma unroll
                    for (int it = 0; it < 4; ++it) ao[it] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int it = 0; it < 4; ++it)
                            ao[it] = mfma32(SB[s], *reinterpret_cast<const f16x8*>(&sQt[(16 * it + m) * RS16 + 32 * s + 8 * g]),
                                            ao[it]);
#pragma unroll
                    for (int s = 0; s < 2; ++s)
#pragma unroll
                        for (int it = 2 * s; it < 4; ++it)
                            ao[it] = mfma32(VB[s], *reinterpret_cast<const f16x8*>(&sAq[(16 * it + m) * RS16S + 32 * s + 8 * g]),
                                            ao[it]);
#pragma unroll
                    for (int it = 0; it < 4; ++it) {
                        const u32x2 o = {f2bf2(p.scale * ao[it][0], p.scale * ao[it][1]),
                                         f2bf2(p.scale * ao[it][2], p.scale * ao[it][3])};
                        if (16 * it + m < L)
                            *reinterpret_cast<u32x2*>(p.out + ((int64_t)t0 + 16 * it + m) * p.out_rs + (int64_t)h * D +
                                                      16 * w + 4 * g) = o;
                    }
                }
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) {
                    const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sF[F_DEC * 128 + 16 * dt + 4 * g]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) S[dt][e] *= d4[e];
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        const f16x8 A = *reinterpret_cast<const f16x8*>(&sKd[(16 * dt + (m ^ dt)) * RS16S + 32 * s + 8 * g]);
                        S[dt] = mfma32(A, VB[s], S[dt]);
                        if (PREC) S[dt] = mfma32(A, VL[s], S[dt]);
                    }
                }
            }
            // checkpoints at chunk boundaries, counted in chunks of the whole sequence
            const int cs = first + cl + 1;
            if (fix) {  // the pair (S_loc, P) of this chunk boundary; the row is composed once S_start is known
                int wsl = -1;
                if (ck_mode == 1 && cs == ck_single) wsl = cur.e[C_CKWS1];
                if (ck_mode == 2 && every > 0 && cs % every == 0 && cs < seqch)
                    wsl = cur.e[C_CKWS] + cs / every - (first / every + 1);
                if (wsl >= 0) {
                    store_state(ws_ck + ((int64_t)(2 * wsl) * H + h) * D * D, S, w, g, m);
                    store_state(ws_ck + ((int64_t)(2 * wsl + 1) * H + h) * D * D, Pm, w, g, m);
                }
            } else {
                if (ck_mode == 1 && cs == ck_single) ck_store(ck_idx[n]);
                if (ck_mode == 2 && every > 0 && cs % every == 0 && cs < seqch) ck_store(ck_idx[ck_row0 + cs / every]);
            }
            // no barrier here: the walk writes no LDS (its outputs go straight to `out`) and reads none of what the
            // next chunk's raw-row phase writes (raw v rows, gate rows, beta); the barrier after that phase orders
            // everything the walk reads before the cumsum and factors overwrite it
        }
        if (fix) {  // the piece's local end state (blocked order) and transition (fp16) for the scan; LDS is free now
            float* st0 = reinterpret_cast<float*>(lds);
            float* st1 = st0 + D * RS32;
            lds_barrier();  // every wave has finished the walk's LDS reads
            stage_state(st0, S, w, g, m);
            stage_state(st1, Pm, w, g, m);
            lds_barrier();
            copy_staged_blocked(ws_h, st0);
            copy_staged_h(reinterpret_cast<half_t*>(ws_h + ws_arr), st1);
            return;
        }
        if (P1 && (pflags & PIECE_STORE_END)) {  // the first piece of a split sequence: the second piece's start state
            store_state(p.ws + 2 * ws_arr + ((int64_t)(slot + 1) * H + h) * D * D, S, w, g, m);
            return;
        }
        // ---- final state (the last piece of a sequence)
        if (pflags & PIECE_LAST) {
            if (pool) {
                if (cur.row >= 0 && cur.row < p.state_slots)
                    store_state(p.state_pool + cur.row * p.state_ss + (int64_t)h * D * D, S, w, g, m);
            } else {
                store_state(p.final_state + ((int64_t)n * H + h) * D * D, S, w, g, m);
            }
        }
        if (!more) break;
        // ---- the next item.  Its rows and dt_bias came in during this item's last chunk, unless this item had none.
        const bool prefetched = nch > 0;
        cur = load_item(++kpos);
        if (!prefetched) {
            load_row<RG>(p, cur.h, cur.tstart, cur.nch > 0 ? min(64, cur.len) : 0, r, cb, RB, nx);
            if (RG && threadIdx.x < D) sDT[threadIdx.x] = dtb_next;
            lds_barrier();
        }
        load_start_state(state_source(cur));
        if (RG) An = gate_an(cur.alog);
    }  // the workgroup's items
}

// Row-block composition used by the scan and the checkpoint compose: out[v][k] = L[v][k] + sum_k' X[v][k'] P[k'][k]
// in fp32, P as the chunk kernel stores it ([k'][k]).  Row v of the result depends on row v of X alone, so one
// workgroup of 256 threads takes a block of 16 rows (grid: entries x H x 8, the 8 blocks of one state on one XCD so
// that P is fetched into one L2).  The product runs on fp32 MFMAs (16x16x4): wave w owns the columns 32 w .. 32 w + 31
// as two 16-column tiles, tile ct holding the columns 32 w + 2 j + ct (j = lane % 16), so that a lane's two B values
// for one k' are one 8-byte load.  MFMA step s covers k' = 32 (lane / 16) + s; a lane's A values (X rows from LDS,
// row stride 132 floats) are 4 consecutive floats per LDS read.  The B values and the L values of one composition
// are loaded into registers ahead of it (ComposeOps), so the scan fetches the next piece's operands while it
// composes the current one.  Result lane layout: rows 4 (lane / 16) + e of the block, columns 32 w + 2 j + {0, 1}.
constexpr int SC_THREADS = 256;
constexpr int SC_ROWS = 16;
constexpr int SC_XS = 132;
constexpr int SC_BUF = SC_ROWS * SC_XS;     // floats of one staged row block
constexpr int SC_SMEM = 2 * SC_BUF * 4;     // two row blocks (the scan alternates between them)

struct ComposeOps {
    f32x2 b[32];  // P[32 kq + s][32 w + 2 j + {0, 1}], s = 0 .. 31
    f32x2 l[4];   // L[4 kq + e][32 w + 2 j + {0, 1}], e = 0 .. 3
};
__device__ __forceinline__ int compose_col() { return 32 * (threadIdx.x >> 6) + 2 * (threadIdx.x & 15); }
__device__ __forceinline__ int compose_row0() { return 4 * ((threadIdx.x & 63) >> 4); }

// the 16 rows starting at X (row stride D) -> sX
__device__ __forceinline__ void stage_X(const float* __restrict__ X, float* sX) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = threadIdx.x + SC_THREADS * j, rr = i >> 5, c4 = i & 31;
        *reinterpret_cast<f32x4*>(sX + rr * SC_XS + 4 * c4) = *reinterpret_cast<const f32x4*>(X + rr * D + 4 * c4);
    }
}
// this lane's operands of one composition: P (a whole state, [k'][k]) and Lblk (the block's first row of L)
__device__ __forceinline__ void fetch_ops(const float* __restrict__ P, const float* __restrict__ Lblk, ComposeOps& o) {
    const int col = compose_col(), r0 = compose_row0();
    const float* pc = P + (8 * r0) * D + col;  // row 32 kq
#pragma unroll
    for (int s = 0; s < 32; ++s) o.b[s] = *reinterpret_cast<const f32x2*>(pc + s * D);
#pragma unroll
    for (int e = 0; e < 4; ++e) o.l[e] = *reinterpret_cast<const f32x2*>(Lblk + (r0 + e) * D + col);
}
// acc[ct][e] = out[4 kq + e][32 w + 2 j + ct]; sX staged and synced
__device__ __forceinline__ void compose_ops(const float* sX, const ComposeOps& o, f32x4 (&acc)[2]) {
    const int j = threadIdx.x & 15, kq = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        acc[0][e] = o.l[e][0];
        acc[1][e] = o.l[e][1];
    }
#pragma unroll
    for (int s4 = 0; s4 < 8; ++s4) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(sX + j * SC_XS + 32 * kq + 4 * s4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int s = 4 * s4 + e;
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], o.b[s][0], acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], o.b[s][1], acc[1], 0, 0, 0);
        }
    }
}
// (entry, head, row block) of this workgroup: XCD-contiguous order keeps an entry-head's 8 blocks on one XCD
__device__ __forceinline__ void scan_task(int H, int blk, int nblk, int& ei, int& h, int& rb) {
    const int t = xcd_task(blk, nblk);
    rb = t & 7;
    const int eh = t >> 3;
    ei = eh / H;
    h = eh - ei * H;
}

// The scan's operands: a later piece stores its local end state S_loc in blocked order (element (a, b) at
// ((a / 4) * 128 + b) * 4 + a % 4, a = v) and its transition P[k'][k] as fp16 in groups of 8 rows (copy_staged_h).
// The product X P runs on f16 16x16x32 MFMAs as X_lo P + X_hi P, X held as the fp16 pair hi = RNE(x),
// lo = RNE(x - hi) (22 bits of mantissa; the state's fp16 range is the walk's own), P as the walk formed it (an fp16
// operand at each of its chunks).  The step is bound by moving its operands into the CU, not by its 16 MFMAs per wave:
// P as one fp16 array is 32 KiB a step against 64 KiB as a bf16 pair.  4 waves per workgroup, wave w on the two
// 16-column tiles 32 w + 16 ct + j; MFMA t covers k' = 32 t + 8 kq .. + 7 (kq = lane / 16, j = lane % 16), so a
// lane's B values per MFMA are one 16-byte load, with the 16 lanes of a row group reading 256 contiguous bytes, and
// its L values (rows 16 rb + 4 kq .. + 3 of S_loc) one more 16-byte load.  The running state block X sits in LDS as
// the fp16 pair (16 hi rows, then 16 lo rows, SCAN_XS halves per row: the 16-byte A reads of the 16 rows fall on
// distinct banks).  One register set of operands is 40 VGPRs.
constexpr int SCAN_THREADS = 256;
constexpr int SCAN_XS = 136;
constexpr int SCAN_XBUF = 2 * SC_ROWS * SCAN_XS;  // halves of one staged block
constexpr int SCAN_SMEM = 2 * SCAN_XBUF * 2;      // two blocks (the scan alternates between them)
struct ScanOps {
    u32x4 b[2][4];  // b[ct][t] = P[32 t + 8 kq .. + 7][32 w + 16 ct + j]
    f32x4 l[2];     // l[ct] = L[16 rb + 4 kq .. + 3][32 w + 16 ct + j]
};
// the fp16 pair hi = RNE(x), lo = RNE(x - hi) of two fp32 values, each pair packed in one word (element 0 low)
__device__ __forceinline__ void split_f16x2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
    const half_t h0 = (half_t)x0, h1 = (half_t)x1;
    const half_t l0 = (half_t)(x0 - (float)h0), l1 = (half_t)(x1 - (float)h1);
    hi = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
    lo = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
}
// Buffer loads: the lane part of the address is one VGPR, the steps between a lane's operand groups are scalar
// offsets (a global load's immediate offset does not reach them, and 64-bit addresses per load cost VGPRs).
// live = false loads nothing (descriptors of no records: the loads return zeros and move no data).
__device__ __forceinline__ void fetch_scan(const float* PB, const float* LB, int rb, bool live, ScanOps& o) {
    const int j = threadIdx.x & 15, kq = (threadIdx.x & 63) >> 4, w = threadIdx.x >> 6;
    const int nrec = __builtin_amdgcn_readfirstlane(live ? D * D * 4 : 0);
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(PB), (short)0, nrec, 0x00020000);
    const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(LB), (short)0, nrec, 0x00020000);
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const int col = 32 * w + 16 * ct + j;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            o.b[ct][t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, (kq * D + col) * 16,
                                                                                         t * 4 * D * 16, 0));
        o.l[ct] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rl, ((4 * rb + kq) * D + col) * 16, 0, 0));
    }
}
// acc[ct][e] = out[4 kq + e][32 w + 16 ct + j]; sX (the fp16 pair block) staged and synced
__device__ __forceinline__ void compose_scan(const uint16_t* sX, const ScanOps& o, f32x4 (&acc)[2]) {
    const int j = threadIdx.x & 15, kq = (threadIdx.x & 63) >> 4;
    acc[0] = o.l[0];
    acc[1] = o.l[1];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const f16x8 ah = *reinterpret_cast<const f16x8*>(sX + j * SCAN_XS + 32 * t + 8 * kq);
        const f16x8 al = *reinterpret_cast<const f16x8*>(sX + (SC_ROWS + j) * SCAN_XS + 32 * t + 8 * kq);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const f16x8 b = __builtin_bit_cast(f16x8, o.b[ct][t]);
            acc[ct] = mfma32(al, b, acc[ct]);
            acc[ct] = mfma32(ah, b, acc[ct]);
        }
    }
}

// Split sequences: X_1 = the first piece's end state (stored by that piece), X_{p+1} = P_p X_p + S_loc(p) for the
// later pieces p = 1 .. np-1; X_p is the start state of piece p, X_np the sequence's final state.  One workgroup per
// (sequence, head, block of 16 state rows).  X_p sits in LDS buffer (p - 1) % 2: step p reads one buffer and writes
// the other, so one barrier per step orders both (a wave writes buffer p % 2 only after every wave has passed step
// p's barrier, i.e. finished reading that buffer in step p - 1).  The barrier covers LDS only: the global stores of
// the states are not waited for.  A freshly written transition takes about two compositions to arrive, so each
// piece's operands are fetched two steps ahead, into one of three register sets (refilled right after the step that
// used it, behind that step's state stores, so that a wait for a store never waits for a prefetch).
// LEAN (every split sequence in at most 3 pieces, config 1's case): one register set, no fetch ahead; ~70 registers fit
// four workgroups per CU, so a launch of many short scans runs in one round.
template <bool LEAN>
__device__ __forceinline__ void scan_body(const PfParams& p, const int32_t* __restrict__ tab, unsigned char* lds, int wg,
                                          int nwg) {
    uint16_t* sX = reinterpret_cast<uint16_t*>(lds);
    const int H = p.H;
    int si, h, rb;
    scan_task(H, wg, nwg, si, h, rb);
    const int32_t* e = tab + tab[H_OFF_SCAN] + S_WORDS * si;
    const int n = e[S_SEQ], np = e[S_NP], slot0 = e[S_SLOT0];
    const int64_t ws_arr = (int64_t)tab[H_NSLOTS] * H * D * D;
    const int j = threadIdx.x & 15, kq = (threadIdx.x & 63) >> 4, w = threadIdx.x >> 6;
    const int64_t blk = (int64_t)SC_ROWS * rb * D;  // the block's first element in a state
    float* fin = nullptr;  // the final state's destination (same rules as the chunk walk)
    if (p.flags & KDA355_PF_POOL) {
        const int64_t row = p.state_idx[n];
        if (row >= 0 && row < p.state_slots) fin = p.state_pool + row * p.state_ss + (int64_t)h * D * D;
    } else {
        fin = p.final_state + ((int64_t)n * H + h) * D * D;
    }
    // piece pc's operands: P at array 1, S_loc at array 0 of the workspace (both in blocked order)
    auto fetch = [&](int pc, ScanOps& o) {
        const int64_t so = ((int64_t)(slot0 + min(pc, np - 1)) * H + h) * D * D;
        fetch_scan(p.ws + ws_arr + so, p.ws + so, rb, pc < np, o);
    };
    // step pc: X_{pc+1} = P_pc X_pc + S_loc(pc) from `o`, which then receives piece pc + 3's operands.  Every step
    // issues the same memory operations, and the loop runs whole groups of three steps: fetches past the last piece
    // and the stores of a step past the last one (or of a missing final-state destination) go through descriptors
    // of no records, so they move no data (a sequence in two pieces, config 1's case, loads one operand set, not
    // three).  With no operation under a branch, the wait for `o` counts only the operations issued after it.
    auto step = [&](int pc, ScanOps& o) {
        lds_barrier();  // X_pc is complete in its buffer
        f32x4 acc[2];
        compose_scan(sX + ((pc - 1) & 1) * SCAN_XBUF, o, acc);
        uint16_t* sN = sX + (pc & 1) * SCAN_XBUF;
        const float* dst = (pc + 1 < np) ? p.ws + 2 * ws_arr + ((int64_t)(slot0 + pc + 1) * H + h) * D * D
                                         : (pc + 1 == np ? fin : nullptr);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            uniform_ptr(dst ? dst : p.ws), (short)0, dst ? D * D * 4 : 0, 0x00020000);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int ee = 0; ee < 4; ++ee) {
                const int rr = 4 * kq + ee, col = 32 * w + 16 * ct + j;
                const half_t hh = (half_t)acc[ct][ee];
                sN[rr * SCAN_XS + col] = __builtin_bit_cast(uint16_t, hh);
                sN[(SC_ROWS + rr) * SCAN_XS + col] = __builtin_bit_cast(uint16_t, (half_t)(acc[ct][ee] - (float)hh));
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[ct][ee]), rs, (int)(blk + rr * D + col) * 4, 0,
                                                      0);
            }
        if constexpr (!LEAN) fetch(pc + 3, o);
    };
    // X_1's 16 rows (one 16-byte piece per thread) are loaded first, then the first three pieces' operands; the
    // LDS write of X_1 then waits for X_1 alone (the compiler barriers keep the loads in this order)
    const float* X1 = p.ws + 2 * ws_arr + ((int64_t)(slot0 + 1) * H + h) * D * D + blk;
    f32x4 x1[2];  // two 16-byte pieces per thread: piece i = threadIdx.x + 256 q -> row i / 32, columns 4 (i % 32)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int i = threadIdx.x + SCAN_THREADS * q;
        x1[q] = *reinterpret_cast<const f32x4*>(X1 + (i >> 5) * D + 4 * (i & 31));
    }
    asm volatile("" ::: "memory");
    if constexpr (LEAN) {
        ScanOps oa;
        fetch(1, oa);
        asm volatile("" ::: "memory");
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int i = threadIdx.x + SCAN_THREADS * q, rr = i >> 5, c = 4 * (i & 31);
            uint32_t h0, l0, h1, l1;
            split_f16x2(x1[q][0], x1[q][1], h0, l0);
            split_f16x2(x1[q][2], x1[q][3], h1, l1);
            *reinterpret_cast<u32x2*>(sX + rr * SCAN_XS + c) = u32x2{h0, h1};
            *reinterpret_cast<u32x2*>(sX + (SC_ROWS + rr) * SCAN_XS + c) = u32x2{l0, l1};
        }
        step(1, oa);
        if (np == 3) {
            fetch(2, oa);
            step(2, oa);
        }
        return;
    }
    ScanOps oa, ob, oc;
    fetch(1, oa);
    fetch(2, ob);
    fetch(3, oc);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int i = threadIdx.x + SCAN_THREADS * q, rr = i >> 5, c = 4 * (i & 31);
        uint32_t h0, l0, h1, l1;
        split_f16x2(x1[q][0], x1[q][1], h0, l0);
        split_f16x2(x1[q][2], x1[q][3], h1, l1);
        *reinterpret_cast<u32x2*>(sX + rr * SCAN_XS + c) = u32x2{h0, h1};
        *reinterpret_cast<u32x2*>(sX + (SC_ROWS + rr) * SCAN_XS + c) = u32x2{l0, l1};
    }
    for (int pc = 1; pc < np; pc += 3) {
        step(pc, oa);
        step(pc + 1, ob);
        step(pc + 2, oc);
    }
}
template <bool LEAN>
__global__ void __launch_bounds__(SCAN_THREADS) scan_kernel(PfParams p, const int32_t* __restrict__ tab) {
    extern __shared__ __align__(16) unsigned char lds[];
    scan_body<LEAN>(p, tab, lds, (int)blockIdx.x, (int)gridDim.x);
}

// Checkpoints inside later pieces: row = P_c S_start + S_loc(c) (fp32), then stored like the chunk walk's checkpoints.
// One workgroup per (task, head, block of 16 state rows); tasks of the checkpoint kind the launch does not use exit.
__device__ __forceinline__ void ck_body(const PfParams& p, const int32_t* __restrict__ tab, unsigned char* lds, int wg,
                                        int nwg) {
    float* sX = reinterpret_cast<float*>(lds);
    const int H = p.H;
    int ti, h, rb;
    scan_task(H, wg, nwg, ti, h, rb);
    const int32_t* e = tab + tab[H_OFF_CKC] + K_WORDS * ti;
    const int ck_mode = (p.flags & KDA355_PF_CK_EVERY) ? 2 : ((p.flags & KDA355_PF_CK_SINGLE) ? 1 : 0);
    if (e[K_KIND] != ck_mode) return;
    const int64_t ws_arr = (int64_t)tab[H_NSLOTS] * H * D * D;
    const float* ws_ck = p.ws + 3 * ws_arr;
    const int col = compose_col(), r0 = compose_row0();
    const int64_t blk = (int64_t)SC_ROWS * rb * D;
    ComposeOps o;
    fetch_ops(ws_ck + ((int64_t)(2 * e[K_WSSLOT] + 1) * H + h) * D * D,
              ws_ck + ((int64_t)(2 * e[K_WSSLOT]) * H + h) * D * D + blk, o);
    stage_X(p.ws + 2 * ws_arr + ((int64_t)e[K_SSLOT] * H + h) * D * D + blk, sX);
    lds_barrier();
    f32x4 acc[2];
    compose_ops(sX, o, acc);
    const int64_t rr = p.ck_idx[e[K_CKIDX]];
    if (rr < 0 || rr >= p.ck_slots) return;
    const int64_t off = rr * p.ck_ss + (int64_t)h * D * D + blk;
#pragma unroll
    for (int ee = 0; ee < 4; ++ee) {
        const int64_t o2 = off + (r0 + ee) * D + col;
        if (p.ck_bf16)
            *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(p.ck_pool) + o2) = f2bf2(acc[0][ee], acc[1][ee]);
        else
            *reinterpret_cast<f32x2*>(reinterpret_cast<float*>(p.ck_pool) + o2) = f32x2{acc[0][ee], acc[1][ee]};
    }
}

// The outputs of later pieces: O = partial (fp16, as the chunk kernel left it in `out`) + scale R S_start, stored as
// bf16.  One workgroup of 256 threads (4 waves) per (group of up to FX_GROUP chunks of one piece, head): the start
// state goes to LDS once per group (fp16 [v][k], rows of 17 16-byte slots, slot s of row v stored at s ^ 4 (v / 32)
// so that the A-fragment reads below hit 16 distinct slots).  Wave w takes tokens 16 w .. 16 w + 15 of every chunk:
// 16x16x32 f16 MFMAs with the state as the A operand (tile vt, A row i <-> value 32 (i / 4) + 4 vt + i % 4) and the R
// rows as the B operand, so lane (g, m) ends with the 32 consecutive values 32 g .. 32 g + 31 of token 16 w + m (four
// 16-byte loads of the partial and four stores).  Each chunk's R rows and partials are loaded one chunk ahead, through
// buffer descriptors that end at the group's last token and last R tile: rows past them read zeros and their stores
// are dropped, so no access sits under a branch.
constexpr int FX_THREADS = 256;
constexpr int FX_GROUP = 2;  // measured: 2 chunks per group beats 1, 4 and 8 (start-state reads vs. tail)
constexpr int FX_ROW = 17 * 16;        // bytes per fp16 state row in LDS
constexpr int FX_SMEM = D * FX_ROW;
__device__ __forceinline__ int fx_slot(int v, int s) { return v * FX_ROW + 16 * (s ^ (4 * (v >> 5))); }
__device__ __forceinline__ void fixup_body(const PfParams& p, const int32_t* __restrict__ tab, unsigned char* lds,
                                           int blk) {
    const int H = p.H;
    const int ti = blk / H;
    const int h = blk - ti * H;
    const int32_t* e = tab + tab[H_OFF_FIX] + X_WORDS * ti;
    const int tstart = e[X_TSTART], L = e[X_LEN];
    const int64_t ws_arr = (int64_t)tab[H_NSLOTS] * H * D * D;
    const float* Sst = p.ws + 2 * ws_arr + ((int64_t)e[X_SSLOT] * H + h) * D * D;  // V-major [v][k]
    const half_t* R0 = reinterpret_cast<const half_t*>(p.ws + 3 * ws_arr + (int64_t)tab[H_NCKSLOTS] * 2 * H * D * D) +
                       ((int64_t)e[X_RSLOT] * H + h) * (64 * D);                  // [token][k], chunk c at + c H 64 D
    const int64_t rstep = (int64_t)H * 64 * D;
    f32x4 x[16];  // S_start, 4 values at a time (v = i / 32, k = 4 (i % 32))
#pragma unroll
    for (int j = 0; j < 16; ++j) x[j] = reinterpret_cast<const f32x4*>(Sst)[threadIdx.x + FX_THREADS * j];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, m = lane & 15, g = lane >> 4;
    const int rs = p.out_rs * 2;  // bytes per output row
    const int tok = 16 * w + m;   // this lane's token inside a chunk
    const __amdgpu_buffer_rsrc_t ob = __builtin_amdgcn_make_buffer_rsrc(
        p.out + (int64_t)tstart * p.out_rs + (int64_t)h * D, (short)0, (L - 1) * rs + D * 2, 0x00020000);
    const int nchk = (L + 63) >> 6;
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<half_t*>(R0), (short)0, (int)((nchk - 1) * rstep * 2 + 64 * D * 2), 0x00020000);
    const int roff = (tok * D + 8 * g) * 2, col = 64 * g;
    // one chunk's operands of this lane: R row tok (k = 32 ks + 8 g .. + 7) and the partial values 32 g .. + 31
    struct Ops { f16x8 X[4]; f16x8 part[4]; };
    auto load = [&](Ops& b, int c0) {
        const int rbase = (int)((c0 >> 6) * rstep * 2) + roff;
        const int obase = (c0 + tok) * rs + col;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            b.X[i] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rb, rbase + 64 * i, 0, 0));
            b.part[i] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(ob, obase + 16 * i, 0, 0));
        }
    };
    // wait for b's loads here (later loads stay in flight) and keep the next chunk's loads above this point
    auto ready = [&](Ops& b) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            asm volatile("" : "+v"(b.X[i])::"memory");
            asm volatile("" : "+v"(b.part[i])::"memory");
        }
    };
    auto finish = [&](const Ops& b, int c0) {
        f32x4 acc[8];
#pragma unroll
        for (int vt = 0; vt < 8; ++vt) {
            acc[vt] = f32x4{0.f, 0.f, 0.f, 0.f};
            const int v = 32 * (m >> 2) + 4 * vt + (m & 3);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                acc[vt] = mfma32(*reinterpret_cast<const f16x8*>(lds + fx_slot(v, 4 * ks + g)), b.X[ks], acc[vt]);
        }
        const int obase = (c0 + tok) * rs + col;
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // values 32 g + 8 i .. + 7 = tiles 2 i and 2 i + 1
            const f16x8& pt = b.part[i];
            const f32x4& a0 = acc[2 * i];
            const f32x4& a1 = acc[2 * i + 1];
            u32x4 r;
            r.x = f2bf((float)pt[0] + p.scale * a0[0]) | (f2bf((float)pt[1] + p.scale * a0[1]) << 16);
            r.y = f2bf((float)pt[2] + p.scale * a0[2]) | (f2bf((float)pt[3] + p.scale * a0[3]) << 16);
            r.z = f2bf((float)pt[4] + p.scale * a1[0]) | (f2bf((float)pt[5] + p.scale * a1[1]) << 16);
            r.w = f2bf((float)pt[6] + p.scale * a1[2]) | (f2bf((float)pt[7] + p.scale * a1[3]) << 16);
            __builtin_amdgcn_raw_buffer_store_b128(r, ob, obase + 16 * i, 0, 0);
        }
    };
    // each chunk's loads are issued one chunk ahead; the loop is unrolled whole (straight-line waits).  The first
    // chunk's loads follow the start state's at once, and the barrier after the start state's LDS writes waits for
    // LDS alone, so they stay in flight through the conversion.
    Ops A, B;
    load(A, 0);
#pragma unroll
    for (int j = 0; j < 16; ++j) {  // S_start -> LDS fp16
        const int i = threadIdx.x + FX_THREADS * j, v = i >> 5, c4 = i & 31;
        const f16x4 hv = {(half_t)x[j][0], (half_t)x[j][1], (half_t)x[j][2], (half_t)x[j][3]};
        *reinterpret_cast<f16x4*>(lds + fx_slot(v, c4 >> 1) + 8 * (c4 & 1)) = hv;
    }
    lds_barrier();
#pragma unroll
    for (int i = 0; i < FX_GROUP; i += 2) {
        if (i + 1 < FX_GROUP) load(B, 64 * (i + 1));
        ready(A);
        finish(A, 64 * i);
        if (64 * (i + 1) >= L) break;
        if (i + 2 < FX_GROUP) load(A, 64 * (i + 2));
        ready(B);
        finish(B, 64 * (i + 1));
        if (64 * (i + 2) >= L) break;
    }
}
// The passes after the scan in one launch: workgroups [0, nscan) run the lean scan (nscan > 0 only when every split
// sequence has 2 pieces, as in config 1: then the fixups and checkpoints need only the first pieces' end states,
// which the chunk kernel stored), the next nfix the output fixup, the rest the checkpoint compose.  Fixups and
// checkpoints are independent of each other: each reads start states and writes its own rows.  Held to 3 waves per
// SIMD (three workgroups per CU instead of four): the fixup then gets registers to keep more of its loads in flight,
// and the HBM-bound rows run 1-2 % faster (config 2 3.35 -> 3.28 ms, p_1x64k 736 -> 728 us).
__global__ void __launch_bounds__(FX_THREADS) __attribute__((amdgpu_waves_per_eu(3, 3))) tail_kernel(PfParams p, const int32_t* __restrict__ tab, int nscan, int nfix) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int b = (int)blockIdx.x;
    if (b < nscan)
        scan_body<true>(p, tab, lds, b, nscan);
    else if (b < nscan + nfix)
        fixup_body(p, tab, lds, b - nscan);
    else
        ck_body(p, tab, lds, b - nscan - nfix, (int)gridDim.x - nscan - nfix);
}

template <bool RG, bool P1, bool PREC>
hipError_t launch_chunk(const PfParams& p, int list_off, int wgs, hipStream_t s) {
    static bool attr_set = false;  // idempotent; a race only repeats the call
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&chunk_kernel<RG, P1, PREC>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, LDS_TOTAL);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL((chunk_kernel<RG, P1, PREC>), dim3(wgs), dim3(PF_THREADS), LDS_TOTAL, s, p, p.tab, p.ck_idx,
                       list_off);
    return hipGetLastError();
}
template <bool P1>
hipError_t launch_chunk_any(const PfParams& p, bool rg, bool prec, int list_off, int wgs, hipStream_t s) {
    return rg ? (prec ? launch_chunk<true, P1, true>(p, list_off, wgs, s) : launch_chunk<true, P1, false>(p, list_off, wgs, s))
              : (prec ? launch_chunk<false, P1, true>(p, list_off, wgs, s) : launch_chunk<false, P1, false>(p, list_off, wgs, s));
}
#include "chunk32.h"

template <typename K>
hipError_t launch_composer(K kernel, const PfParams& p, int entries, int threads, int smem, hipStream_t s,
                           bool& attr_set) {
    if (!attr_set) {  // idempotent; a race only repeats the call
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, smem);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL(kernel, dim3(entries * p.H * (D / SC_ROWS)), dim3(threads), smem, s, p, p.tab);
    return hipGetLastError();
}
hipError_t launch_scan(const PfParams& p, int entries, bool lean, hipStream_t s) {
    static bool attr_set[2] = {false, false};
    return lean ? launch_composer(scan_kernel<true>, p, entries, SCAN_THREADS, SCAN_SMEM, s, attr_set[1])
                : launch_composer(scan_kernel<false>, p, entries, SCAN_THREADS, SCAN_SMEM, s, attr_set[0]);
}
hipError_t launch_tail(const PfParams& p, int scan_entries, int fix_entries, int ck_entries, hipStream_t s) {
    static_assert(SCAN_THREADS == FX_THREADS && SC_THREADS == FX_THREADS && SCAN_SMEM <= FX_SMEM && SC_SMEM <= FX_SMEM,
                  "tail_kernel runs every pass in one launch shape");
    const int nscan = scan_entries * p.H * (D / SC_ROWS), nfix = fix_entries * p.H;
    const int nck = ck_entries * p.H * (D / SC_ROWS);
    if (nscan + nfix + nck == 0) return hipSuccess;
    hipLaunchKernelGGL(tail_kernel, dim3(nscan + nfix + nck), dim3(FX_THREADS), FX_SMEM, s, p, p.tab, nscan, nfix);
    return hipGetLastError();
}

bool aligned(const void* ptr, size_t a) { return (reinterpret_cast<uintptr_t>(ptr) % a) == 0; }

}  // namespace
}  // namespace kda355

using namespace kda355;

// ---------------------------------------------------------------------------------------------------- host plan
extern "C" int kda355_prefill_plan(const KdaPrefillPlanIn* in, KdaPrefillPlan* plan, int32_t* tables, int64_t capacity) {
    KDA_CHECK_ARG(in && plan, "prefill_plan: null argument");
    KDA_CHECK_ARG(in->cu_seqlens, "prefill_plan: cu_seqlens is null");
    const int N = in->N;
    KDA_CHECK_ARG(N >= 1 && in->H >= 1, "prefill_plan: N=%d H=%d", N, in->H);
    const int64_t* cu = in->cu_seqlens;
    KDA_CHECK_ARG(cu[0] == 0, "prefill_plan: cu_seqlens[0] must be 0");
    for (int n = 0; n < N; ++n) KDA_CHECK_ARG(cu[n + 1] >= cu[n], "prefill_plan: cu_seqlens must be non-decreasing");
    const int64_t T = cu[N];
    KDA_CHECK_ARG(T < (1ll << 31) - 64, "prefill_plan: too many tokens");
    KDA_CHECK_ARG(in->ck_every >= 0 && in->ck_every % KDA355_CHUNK == 0, "prefill_plan: ck_every must be a multiple of 64");
    const int every_chunks = in->ck_every / KDA355_CHUNK;
    std::vector<int> nch(N);
    int64_t nchunks = 0;
    for (int n = 0; n < N; ++n) {
        nch[n] = (int)((cu[n + 1] - cu[n] + 63) / 64);
        nchunks += nch[n];
    }
    // Pieces.  A workgroup walks one (piece, head) chain and a CU holds one such workgroup at a time; the chain list is
    // dispatched longest first.  Candidate cuts: every sequence longer than a piece length T is cut into
    // ceil(nch / T) near-equal pieces, or into pieces of T chunks followed by the remainder (which fills CUs the long
    // pieces leave idle: 16 chunks on 3/4 of the CUs cut as 12 + 4), for T on a geometric ladder from a quarter of the
    // balanced per-CU load.  Pieces have >= MIN_PIECE chunks in a first pass and >= 1 in a second, whose candidates
    // must beat the first pass's best.  Each candidate is costed in chunk times (one chunk of one head on one CU,
    // ~11 us) by list-scheduling its workgroups in launch order onto the CUs of the shader engine each one is sent to
    // (later pieces cost as much per chunk as first ones), plus the passes a split adds: the scan, sequential over the
    // pieces of a sequence (SCAN_BASE + STEP_UNITS per later piece of the most-cut sequence, + SCAN_WG_UNITS per scan
    // workgroup per CU: 8 per split sequence and head), and the output fixup (FIX_BASE + FIX_UNITS per chunk-head of
    // later pieces, spread over the chip); every workgroup also pays a start-up of START_QUARTERS / 4 chunk times.  The cheapest candidate wins; ties keep fewer pieces.  The
    // first piece of a split sequence runs from the true start state; later pieces run from S = 0, carry their
    // transition and are completed by the scan, fixup and checkpoint-compose kernels.  Measured on MI355X: the scan
    // ~7 us to start and ~0.55 us a step, the fixup ~11 ns per chunk-head.
    constexpr int MIN_PIECE = 2;  // the shortest piece of the first pass (the second allows one chunk)
    constexpr double SCAN_BASE = 0.6, STEP_UNITS = 0.05, SCAN_WG_UNITS = 0.25, FIX_BASE = 0.5, FIX_UNITS = 0.0012;
    constexpr int64_t START_QUARTERS = 4;  // a workgroup's start-up (state, first rows): about one chunk time
    const int num_cus = in->num_cus > 0 ? in->num_cus : 256;
    // MI355X: 8 XCDs of 4 shader engines of 8 CUs; workgroup i goes to XCD i % 8 and, dealt round-robin over the
    // XCD's engines, to the group of workgroups j == i (mod 32)
    const int ngrp = (num_cus >= 32 && num_cus % 32 == 0) ? 32 : 1, cus_per_grp = num_cus / ngrp;
    // chunk counts of the pieces of a c-chunk sequence for piece length T and shortest piece minp: near-equal (mode 0),
    // or T chunks each and the remainder last (mode 1; a remainder under minp joins the piece before it)
    auto piece_lengths = [](int c, int T, int mode, int minp, std::vector<int>& out) {
        out.clear();
        if (c <= T || c < 2 * minp) {
            out.push_back(c);
        } else if (mode == 0) {
            const int np = std::max(1, std::min(c / minp, (c + T - 1) / T));
            for (int pc = 0; pc < np; ++pc) out.push_back(c / np + (pc < c % np ? 1 : 0));
        } else {
            int left = c;
            while (left > T) { out.push_back(T); left -= T; }
            if (left >= minp) out.push_back(left); else out.back() += left;
        }
    };
    int cutT = 1 << 30, cutMode = 0, cutMin = MIN_PIECE;  // no cut unless the cost model finds one
    if (nchunks > 0) {
        int maxc = 0;
        for (int n = 0; n < N; ++n) maxc = std::max(maxc, nch[n]);
        const int64_t avg = std::max<int64_t>(1, (nchunks * in->H + num_cus - 1) / num_cus);
        const bool idle = (int64_t)N * in->H < num_cus;
        if ((idle || 4 * (int64_t)maxc > 5 * avg) && maxc >= 2) {
            std::vector<int> counts, lens;
            std::vector<int64_t> loads;
            const int64_t total_units = nchunks * in->H;
            double best = 0.0;
            auto cost = [&](int T, int mode, int minp, bool first) {
                counts.clear();
                int64_t fixch = 0;
                int nsplit = 0, most = 0, maxnp = 1;
                for (int n = 0; n < N; ++n) {
                    piece_lengths(nch[n], T, mode, minp, lens);
                    const int np = (int)lens.size();
                    maxnp = std::max(maxnp, np);
                    for (int pc = 0; pc < np; ++pc) {
                        const int c = lens[pc];
                        counts.push_back(c);
                        most = std::max(most, c);
                        if (pc > 0) fixch += c;
                    }
                    nsplit += np > 1;
                }
                const double extra =
                    nsplit ? SCAN_BASE + STEP_UNITS * (maxnp - 1) + SCAN_WG_UNITS * 8.0 * nsplit * in->H / num_cus +
                                 FIX_BASE + FIX_UNITS * (double)fixch * in->H
                           : 0.0;
                // loads in quarter chunk times: a workgroup costs its chunks plus its start-up
                const int64_t q_total = 4 * total_units + START_QUARTERS * (int64_t)counts.size() * in->H;
                // no schedule beats the longest piece or the perfect balance
                const double bound =
                    0.25 * (double)std::max<int64_t>(4 * most + START_QUARTERS, (q_total + num_cus - 1) / num_cus) + extra;
                if (!first && bound >= best) return bound;
                std::sort(counts.begin(), counts.end(), std::greater<int>());
                // list scheduling in launch order (chains longest first, heads within a chain): the hardware sends
                // workgroup i to one shader engine (8 CUs) of one XCD, the same for every i of one residue mod 32,
                // and there it takes the CU that frees up first; a workgroup waiting for a CU does not move to
                // another engine, even when CUs elsewhere are idle
                loads.assign(num_cus, 0);  // per engine a min-heap of finish times (all zero: valid heaps)
                int64_t span = 0, wg = 0;
                for (int c : counts)
                    for (int hh = 0; hh < in->H; ++hh, ++wg) {
                        const auto b = loads.begin() + (wg % ngrp) * cus_per_grp, e = b + cus_per_grp;
                        std::pop_heap(b, e, std::greater<int64_t>());
                        *(e - 1) += 4 * c + START_QUARTERS;
                        span = std::max(span, *(e - 1));
                        std::push_heap(b, e, std::greater<int64_t>());
                    }
                return 0.25 * (double)span + extra;
            };
            best = cost(maxc, 0, MIN_PIECE, true);
            // pieces shorter than a quarter of the balanced load per CU only add fixup work: the ladder starts there
            for (int minp = MIN_PIECE; minp >= 1; --minp)
                for (double t = std::max<double>(minp, (double)avg / 4); t < maxc; t *= 1.12) {
                    const int T = (int)t;
                    for (int mode = 0; mode < 2; ++mode) {
                        const double c = cost(T, mode, minp, false);
                        if (c < best - 1e-9) { best = c; cutT = T; cutMode = mode; cutMin = minp; }
                    }
                }
            // then piece lengths within one ladder step of the best (at most ~32 per cut style)
            if (cutT < maxc) {
                const int lo = std::max(cutMin, (int)(cutT / 1.12)), hi = std::min(maxc - 1, (int)(cutT * 1.12) + 1);
                const int T0 = cutT, step = std::max(1, (hi - lo) / 32);
                for (int T = lo; T <= hi; T += step)
                    for (int mode = 0; mode < 2; ++mode) {
                        if (T == T0) continue;
                        const double c = cost(T, mode, cutMin, false);
                        if (c < best - 1e-9) { best = c; cutT = T; cutMode = mode; }
                    }
            }
        }
    }
    std::vector<int> ck_chunk(N, 0), ck_row0(N, 0);
    {
        int64_t ckstart = 0;
        for (int n = 0; n < N; ++n) {
            if (in->ck_offsets) {
                const int32_t o = in->ck_offsets[n];
                // kda/mi350x/kda/prefill/main.cpp:110-118: offsets that are not positive multiples of 64 within the
                // sequence write nothing
                if (o > 0 && o % 64 == 0 && o <= cu[n + 1] - cu[n]) ck_chunk[n] = o / 64;
            }
            ck_row0[n] = (int)ckstart;
            if (every_chunks) ckstart += (nch[n] + every_chunks - 1) / every_chunks;
        }
    }
    struct Piece { int n, first, count, slot, rbase, ckws, ckws1, flags; };
    struct CkTask { int ckidx, wsslot, sslot, kind; };
    std::vector<Piece> pieces;
    std::vector<CkTask> cktasks;
    int nslots = 0, nsplit = 0, nrslots = 0, nfix = 0, nsplitpieces = 0;
    std::vector<int> plens, npieces(N, 1);
    for (int n = 0; n < N; ++n) {
        piece_lengths(nch[n], cutT, cutMode, cutMin, plens);
        const int np = (int)plens.size();
        npieces[n] = np;
        int f = 0;
        for (int pc = 0; pc < np; ++pc) {
            const int c = plens[pc];
            Piece P{n, f, c, np > 1 ? nslots + pc : 0, 0, 0, 0, 0};
            if (np == 1) {
                P.flags = PIECE_LAST;
            } else if (pc == 0) {
                P.flags = PIECE_STORE_END;
            } else {
                P.flags = PIECE_FIX;
                P.rbase = nrslots;
                nrslots += c;
                nfix += (c + FX_GROUP - 1) / FX_GROUP;
                // checkpoints of both kinds the layout defines (the launch's mode uses one): the single one at
                // ck_chunk, every-n rows j at chunk j * every (row 0 is the start state, in the first piece)
                P.ckws1 = (int)cktasks.size();
                if (ck_chunk[n] > f && ck_chunk[n] <= f + c) cktasks.push_back({n, (int)cktasks.size(), P.slot, 1});
                P.ckws = (int)cktasks.size();
                if (every_chunks > 0)
                    for (int j = f / every_chunks + 1; (int64_t)j * every_chunks <= f + c && j * every_chunks < nch[n]; ++j)
                        cktasks.push_back({ck_row0[n] + j, (int)cktasks.size(), P.slot, 2});
            }
            pieces.push_back(P);
            f += c;
        }
        if (np > 1) {
            nslots += np;
            ++nsplit;
            nsplitpieces += np;
        }
    }
    const int nfinal = (int)pieces.size(), nck = (int)cktasks.size();
    // chain list: longest pieces first (they start earliest when the grid runs in several rounds)
    std::vector<int> order(nfinal);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return pieces[a].count > pieces[b].count; });
    // Workgroup lists (unsplit layouts whose (chain, head) items outnumber the CUs): one workgroup per CU walks a list
    // of items in turn, fetching each next item's first rows and start state while the one before it finishes, so
    // only its first item pays the start-up.  Items go in launch order (longest first) to the list with the least work
    // so far.  Costed like the cuts above (one start-up per list, PASS_QUARTERS per later item), the lists are used
    // when their schedule beats one workgroup per item dealt out by the hardware.
    constexpr int64_t PASS_QUARTERS = 1;
    const int64_t items = (int64_t)nfinal * in->H;
    int grid = 0, chunk32 = 0;
    std::vector<std::vector<int32_t>> lists;
    if (nsplit == 0 && items > num_cus && items < (1 << 30)) {
        std::vector<int64_t> ld(num_cus, 0);
        int64_t span_dyn = 0, wg = 0;
        for (int i = 0; i < nfinal; ++i)
            for (int hh = 0; hh < in->H; ++hh, ++wg) {
                const auto b = ld.begin() + (wg % ngrp) * cus_per_grp, e = b + cus_per_grp;
                std::pop_heap(b, e, std::greater<int64_t>());
                *(e - 1) += 4 * pieces[order[i]].count + START_QUARTERS;
                span_dyn = std::max(span_dyn, *(e - 1));
                std::push_heap(b, e, std::greater<int64_t>());
            }
        typedef std::pair<int64_t, int> LoadWg;
        std::priority_queue<LoadWg, std::vector<LoadWg>, std::greater<LoadWg>> q;
        for (int b = 0; b < num_cus; ++b) q.push({0, b});
        lists.assign(num_cus, {});
        int64_t span_lst = 0;
        for (int i = 0; i < nfinal; ++i)
            for (int hh = 0; hh < in->H; ++hh) {
                LoadWg top = q.top();
                q.pop();
                top.first += 4 * pieces[order[i]].count + (lists[top.second].empty() ? START_QUARTERS : PASS_QUARTERS);
                lists[top.second].push_back(i * in->H + hh);
                span_lst = std::max(span_lst, top.first);
                q.push(top);
            }
        if (span_lst < span_dyn) grid = num_cus;
        // The 32-token kernel's schedule (chunk32.h): one workgroup per item, two per CU, items in launch order, the
        // first 2 x num_cus dealt two to a CU and every later one to the CU that frees a slot first.  A workgroup
        // advances C32_PAIRED chunk times per 64 tokens while it shares its CU and C32_ALONE when alone, plus
        // C32_START of start-up, in chunk times of the 64-token kernel.  The constants are a least-squares fit (in
        // log ratio) to eleven layouts timed on MI355X with both kernels: 384-1024 items of 2-32 chunks, where the
        // 32-token kernel runs 3-11 % faster, a ragged layout 8 % slower, the 5-47-chunk p96 layouts 28-35 % slower
        // (long chains alone on their CUs).  It is used when this simulated span beats the 64-token kernel's best
        // (lists or one workgroup per item) by 3 %.
        constexpr double C32_ALONE = 1.2, C32_PAIRED = 1.85, C32_START = 0.3;
        struct Cu { double t = 0, w[2] = {0, 0}; int n = 0, ver = 0; };
        std::vector<Cu> cu(num_cus);
        typedef std::pair<double, std::pair<int, int>> Ev;  // (finish time, (CU, version))
        std::priority_queue<Ev, std::vector<Ev>, std::greater<Ev>> ev;
        int64_t next = 0;
        auto item_work = [&](int64_t it) { return (double)pieces[order[it / in->H]].count + C32_START; };
        auto schedule = [&](int c) {  // the CU's next completion
            Cu& u = cu[c];
            if (u.n == 0) return;
            const double r = u.n == 2 ? C32_PAIRED : C32_ALONE;
            ev.push({u.t + std::min(u.w[0], u.n == 2 ? u.w[1] : u.w[0]) * r, {c, ++u.ver}});
        };
        for (int rnd = 0; rnd < 2; ++rnd)
            for (int c = 0; c < num_cus && next < items; ++c) cu[c].w[cu[c].n++] = item_work(next++);
        for (int c = 0; c < num_cus; ++c) schedule(c);
        // Workgroups that finish at one instant free their slots together; the waiting items go first one to each
        // such CU, then to the CUs that freed a second slot (the hardware spreads a burst over the CUs).
        double span32 = 0;
        std::vector<int> freed[2];
        while (!ev.empty()) {
            const double t = ev.top().first;
            freed[0].clear();
            freed[1].clear();
            while (!ev.empty() && ev.top().first <= t + 1e-9) {
                const Ev e = ev.top();
                ev.pop();
                const int c = e.second.first;
                Cu& u = cu[c];
                if (e.second.second != u.ver) continue;  // superseded by a later change of this CU
                const double r = u.n == 2 ? C32_PAIRED : C32_ALONE;
                double w[2], wmin = 1e300;
                for (int j = 0; j < u.n; ++j) wmin = std::min(wmin, w[j] = u.w[j] - (e.first - u.t) / r);
                int left = 0;  // the event's workgroup finishes whatever the rounding left of its work
                for (int j = 0; j < u.n; ++j)
                    if (w[j] > std::max(1e-9, wmin + 1e-9)) u.w[left++] = w[j];
                for (int j = left; j < u.n; ++j) freed[j - left].push_back(c);
                u.n = left;
                u.t = e.first;
                ++u.ver;
                span32 = std::max(span32, e.first);
            }
            for (int k = 0; k < 2; ++k)
                for (const int c : freed[k])
                    if (next < items) cu[c].w[cu[c].n++] = item_work(next++);
            for (int k = 0; k < 2; ++k)
                for (const int c : freed[k]) schedule(c);  // a CU listed twice is rescheduled twice: the later wins
        }
        if (span32 < 0.97 * 0.25 * (double)std::min(span_lst, span_dyn)) chunk32 = 1;
    }
    const int64_t off_final = H_WORDS, off_fix = off_final + (int64_t)C_WORDS * nfinal;
    const int64_t off_scan = off_fix + (int64_t)X_WORDS * nfix;
    const int64_t off_ckc = off_scan + (int64_t)S_WORDS * nsplit;
    const int64_t off_wg = off_ckc + (int64_t)K_WORDS * nck;
    const int64_t words = off_wg + (grid ? grid + 1 + items : 0);
    plan->T = T;
    plan->N = N;
    plan->H = in->H;
    plan->num_chunks = (int32_t)nchunks;
    plan->num_chains = nfinal;
    int maxc = 0;
    int64_t ckrows = 0;
    for (int n = 0; n < N; ++n) {
        maxc = std::max(maxc, nch[n]);
        if (every_chunks) ckrows += (nch[n] + every_chunks - 1) / every_chunks;
    }
    const int64_t dd = (int64_t)KDA355_HEAD_DIM * KDA355_HEAD_DIM;
    plan->max_chain_chunks = maxc;
    plan->table_words = words;
    plan->workspace_bytes = ((int64_t)3 * nslots + 2 * (int64_t)nck) * in->H * dd * 4 +
                            (int64_t)nrslots * in->H * 64 * KDA355_HEAD_DIM * 2;
    plan->ck_rows = ckrows;
    plan->magic = PLAN_MAGIC;
    plan->flags = in->flags;
    plan->ck_every = in->ck_every;
    plan->num_pieces = nsplitpieces;
    plan->num_split = nsplit;
    plan->num_fix_tasks = nfix;
    plan->num_ck_tasks = nck;
    plan->chunk_grid = grid;
    plan->chunk32 = chunk32;
    if (!tables) return 0;
    KDA_CHECK_ARG(capacity >= words, "prefill_plan: table capacity %lld < %lld words", (long long)capacity, (long long)words);
    int32_t* t = tables;
    std::fill(t, t + words, 0);
    t[H_MAGIC] = (int32_t)PLAN_MAGIC;
    t[H_N] = N;
    t[H_T] = (int32_t)T;
    t[H_NCHUNK] = (int32_t)nchunks;
    t[H_EVERY] = every_chunks;
    t[H_CKROWS] = (int32_t)ckrows;
    t[H_OFF_FINAL] = (int32_t)off_final;
    t[H_NFINAL] = nfinal;
    t[H_OFF_FIX] = (int32_t)off_fix;
    t[H_NFIX] = nfix;
    t[H_OFF_SCAN] = (int32_t)off_scan;
    t[H_NSCAN] = nsplit;
    t[H_NSLOTS] = nslots;
    t[H_OFF_CKC] = (int32_t)off_ckc;
    t[H_NCKC] = nck;
    t[H_NRSLOTS] = nrslots;
    t[H_NCKSLOTS] = nck;
    auto fill = [&](int32_t* e, const Piece& pc) {
        const int64_t len = cu[pc.n + 1] - cu[pc.n];
        e[C_SEQ] = pc.n;
        e[C_NCH] = pc.count;
        e[C_TSTART] = (int32_t)(cu[pc.n] + 64 * (int64_t)pc.first);
        e[C_LEN] = (int32_t)std::max<int64_t>(0, std::min<int64_t>(64 * (int64_t)pc.count, len - 64 * (int64_t)pc.first));
        e[C_CKSINGLE] = ck_chunk[pc.n];
        e[C_CKROW0] = ck_row0[pc.n];
        e[C_FIRST] = pc.first;
        e[C_FLAGS] = pc.flags;
        e[C_SLOT] = pc.slot;
        e[C_SEQCH] = nch[pc.n];
        e[C_RBASE] = pc.rbase;
        e[C_CKWS] = pc.ckws;
        e[C_CKWS1] = pc.ckws1;
    };
    for (int i = 0; i < nfinal; ++i) fill(t + off_final + (int64_t)C_WORDS * i, pieces[order[i]]);
    if (grid) {  // [grid + 1] list starts, then the items of list 0, 1, ...
        t[H_OFF_WG] = (int32_t)off_wg;
        int32_t* ws = t + off_wg;
        int32_t pos = 0;
        for (int b = 0; b < grid; ++b) {
            ws[b] = pos;
            for (int32_t it : lists[b]) ws[grid + 1 + pos++] = it;
        }
        ws[grid] = pos;
    }
    int xi = 0, si = 0;
    for (const Piece& pc : pieces) {
        if (pc.flags & PIECE_FIX) {
            const int64_t len = cu[pc.n + 1] - cu[pc.n];
            for (int c = 0; c < pc.count; c += FX_GROUP) {
                int32_t* e = t + off_fix + (int64_t)X_WORDS * xi++;
                const int64_t c0 = 64 * (int64_t)(pc.first + c);
                e[X_TSTART] = (int32_t)(cu[pc.n] + c0);
                e[X_LEN] = (int32_t)std::min<int64_t>(64 * (int64_t)std::min(FX_GROUP, pc.count - c), len - c0);
                e[X_RSLOT] = pc.rbase + c;
                e[X_SSLOT] = pc.slot;
            }
        }
        if (pc.flags & PIECE_STORE_END) {
            int32_t* e = t + off_scan + (int64_t)S_WORDS * si++;
            e[S_SEQ] = pc.n;
            e[S_NP] = npieces[pc.n];
            e[S_SLOT0] = pc.slot;
        }
    }
    for (int i = 0; i < nck; ++i) {
        int32_t* e = t + off_ckc + (int64_t)K_WORDS * i;
        e[K_CKIDX] = cktasks[i].ckidx;
        e[K_WSSLOT] = cktasks[i].wsslot;
        e[K_SSLOT] = cktasks[i].sslot;
        e[K_KIND] = cktasks[i].kind;
    }
    return 0;
}

extern "C" int64_t kda355_prefill_workspace_bytes(const KdaPrefillPlan* plan) {
    if (!plan || plan->magic != PLAN_MAGIC) return -1;
    return plan->workspace_bytes;
}

extern "C" int kda355_prefill_launch(const KdaPrefillArgs* a, kda355_stream_t stream) {
    KDA_CHECK_ARG(a && a->plan, "prefill: null args or plan");
    const KdaPrefillPlan* pl = a->plan;
    KDA_CHECK_ARG(pl->magic == PLAN_MAGIC, "prefill: plan is not a kda355_prefill_plan() result");
    KDA_CHECK_ARG(pl->chunk_grid >= 0 && (int64_t)pl->chunk_grid <= (int64_t)pl->num_chains * pl->H &&
                      (pl->chunk_grid == 0 || pl->num_split == 0),
                  "prefill: plan has an invalid chunk_grid %d", pl->chunk_grid);
    KDA_CHECK_ARG((pl->chunk32 == 0 || pl->chunk32 == 1) && (pl->chunk32 == 0 || pl->num_split == 0),
                  "prefill: plan has an invalid chunk32 %d", pl->chunk32);
    KDA_CHECK_ARG(pl->N == a->N && pl->T == a->T && pl->H == a->H,
                  "prefill: plan was made for another layout (N/T/H %d/%lld/%d vs %d/%lld/%d)", pl->N, (long long)pl->T,
                  pl->H, a->N, (long long)a->T, a->H);
    const uint32_t f = a->flags;
    KDA_CHECK_ARG(a->q && a->k && a->v && a->g && a->beta && a->out && a->tables, "prefill: a required pointer is null");
    KDA_CHECK_ARG(!(f & KDA355_PF_RAW_GATE) || (a->A_log && a->dt_bias), "prefill: raw gate needs A_log and dt_bias");
    const bool pool = f & KDA355_PF_POOL;
    KDA_CHECK_ARG(pool ? (a->state_pool && a->state_idx && a->has_initial_state) : (a->final_state != nullptr),
                  "prefill: pool mode needs state_pool/state_idx/has_initial_state, contiguous mode final_state");
    KDA_CHECK_ARG(!(f & (KDA355_PF_CK_SINGLE | KDA355_PF_CK_EVERY)) || (a->ck_pool && a->ck_idx),
                  "prefill: checkpoints need ck_pool and ck_idx");
    KDA_CHECK_ARG(!((f & KDA355_PF_CK_EVERY) && (f & KDA355_PF_CK_SINGLE)), "prefill: choose one checkpoint mode");
    KDA_CHECK_ARG(!(f & KDA355_PF_CK_EVERY) || pl->ck_every > 0, "prefill: every-n checkpoints need a plan with ck_every");
    KDA_CHECK_ARG(aligned(a->q, 16) && aligned(a->k, 16) && aligned(a->v, 16) && a->qkv_row_stride % 8 == 0,
                  "prefill: q/k/v rows must be 16-byte aligned");
    // every row piece is moved as 16-byte vectors: 16-byte aligned bases and row strides
    KDA_CHECK_ARG((f & KDA355_PF_RAW_GATE) ? (aligned(a->g, 16) && a->g_row_stride % 8 == 0)
                                           : (aligned(a->g, 16) && a->g_row_stride % 4 == 0),
                  "prefill: g rows must be 16-byte aligned");
    KDA_CHECK_ARG(aligned(a->out, 16) && a->out_row_stride % 8 == 0, "prefill: out rows must be 16-byte aligned");
    // the kernels address the rows of one 64-token chunk with 32-bit offsets
    KDA_CHECK_ARG(a->qkv_row_stride < (1 << 21) && a->g_row_stride < (1 << 21) && a->beta_row_stride < (1 << 21) &&
                      a->out_row_stride < (1 << 21) && a->qkv_row_stride >= 0 && a->g_row_stride >= 0 &&
                      a->beta_row_stride >= 0 && a->out_row_stride >= 0,
                  "prefill: row strides must be in [0, 2^21) elements");
    KDA_CHECK_ARG(!pool || (aligned(a->state_pool, 16) && a->state_slot_stride % 4 == 0), "prefill: state pool misaligned");
    KDA_CHECK_ARG(pool || (aligned(a->final_state, 16) && (!a->initial_state || aligned(a->initial_state, 16))),
                  "prefill: states misaligned");
    KDA_CHECK_ARG(!a->ck_pool || (aligned(a->ck_pool, 16) && a->ck_slot_stride % 8 == 0), "prefill: ck pool misaligned");
    KDA_CHECK_ARG(pl->workspace_bytes == 0 || (a->workspace && aligned(a->workspace, 256)),
                  "prefill: this layout splits sequences and needs a 256-byte aligned workspace of %lld bytes",
                  (long long)pl->workspace_bytes);
    if (a->N == 0) return 0;
    PfParams p;
    p.q = static_cast<const uint16_t*>(a->q);
    p.k = static_cast<const uint16_t*>(a->k);
    p.v = static_cast<const uint16_t*>(a->v);
    p.g = a->g;
    p.beta = a->beta;
    p.A_log = a->A_log;
    p.dt_bias = a->dt_bias;
    p.out = static_cast<uint16_t*>(a->out);
    p.state_pool = a->state_pool;
    p.state_idx = a->state_idx;
    p.has_init = a->has_initial_state;
    p.init_state = a->initial_state;
    p.final_state = a->final_state;
    p.ck_pool = a->ck_pool;
    p.ck_idx = a->ck_idx;
    p.tab = a->tables;
    p.qkv_rs = a->qkv_row_stride;
    p.g_rs = a->g_row_stride;
    p.beta_rs = a->beta_row_stride;
    p.out_rs = a->out_row_stride;
    p.state_ss = a->state_slot_stride;
    p.state_slots = a->state_slots;
    p.ck_ss = a->ck_slot_stride;
    p.ck_slots = a->ck_slots;
    p.N = a->N;
    p.H = a->H;
    p.scale = a->scale;
    p.lb = a->lower_bound;
    p.flags = f;
    p.ck_bf16 = a->ck_dtype == 1;
    p.ws = static_cast<float*>(a->workspace);
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool rg = (f & KDA355_PF_RAW_GATE) != 0;
    const bool prec = (f & KDA355_PF_PRECISE) != 0;
    const int off_final = H_WORDS;
    hipError_t e = hipSuccess;
    if (pl->num_split > 0) {
        // one chunk launch for every piece (first pieces from their true start states, later pieces from zero with their
        // transitions), then the start / final states of the split sequences, the later pieces' outputs and their
        // checkpoints
        e = launch_chunk_any<true>(p, rg, prec, off_final, pl->num_chains * a->H, s);
        // every split sequence has >= 2 pieces, so the most-cut one has at most num_pieces - 2 (num_split - 1)
        const bool lean = pl->num_pieces - 2 * (pl->num_split - 1) <= 3;
        if (pl->num_pieces == 2 * pl->num_split) {  // every split sequence in 2 pieces: the scan joins the tail launch
            if (e == hipSuccess) e = launch_tail(p, pl->num_split, pl->num_fix_tasks, pl->num_ck_tasks, s);
        } else {
            if (e == hipSuccess) e = launch_scan(p, pl->num_split, lean, s);
            if (e == hipSuccess) e = launch_tail(p, 0, pl->num_fix_tasks, pl->num_ck_tasks, s);
        }
    } else {
        // one workgroup per (chain, head), or the plan's workgroup lists; or, when the plan chose it, the 32-token
        // kernel (one workgroup per item, two per CU), outside the precise mode and unless the caller keeps the
        // 64-token kernel (KDA355_PF_CHUNK64)
        const int items = pl->num_chains * a->H;
        if (pl->chunk32 && !prec && !(f & KDA355_PF_CHUNK64))
            e = rg ? launch_chunk32<true>(p, off_final, items, s) : launch_chunk32<false>(p, off_final, items, s);
        else
            e = launch_chunk_any<false>(p, rg, prec, off_final, pl->chunk_grid > 0 ? pl->chunk_grid : items, s);
    }
    if (e != hipSuccess) {
        set_error("prefill: launch failed: %s", hipGetErrorString(e));
        return KDA355_ELAUNCH;
    }
    return 0;
}
