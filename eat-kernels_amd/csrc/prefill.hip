// Chunked KDA prefill on gfx950 (chunk 64, head dim 128): host plan, chunk prologue kernel, chain walk kernel.
//
// Math (per sequence n, head h, chunk of c <= 64 tokens; Gamma = inclusive cumsum of the log-decay g over the chunk,
// per key channel; S the fp32 state, K-major in the formulas, V-major in memory):
//     A_kk = strict_tril(diag(beta) (K e^{Gamma}) (K e^{-Gamma})^T),   A_qk = tril((Q e^{Gamma}) (K e^{-Gamma})^T)
//     T    = (I + A_kk)^-1
//     W    = T diag(beta) (K e^{Gamma}),   U = T diag(beta) V
//     Qp   = Q e^{Gamma} - A_qk W,          Oi = A_qk U                  (so that O = scale (Qp S + Oi))
//     Kd   = K e^{Gamma_c - Gamma},         decay = e^{Gamma_c}
//   per chunk, serially:  V' = U - W S;   O = scale (Qp S + Oi);   S <- diag(decay) S + Kd^T V'
// This is the token recurrence of kda/mi350x/reference.py:85-91 regrouped per chunk (the chunked WY form; the same
// operator as kda/b200/csrc/w3/base/tiny/kda_tiny.cu:5-10 and vLLM's qg / w / u / kg_t / decay decomposition,
// kda/mi350x/benchmark/baselines/prefill/vllm_reference/kda_chunk.py:73-76, 97-108).  Folding A_qk W into Qp takes
// the A_qk V' product off the serial path.
//
// Precision plan (from a numerical model of this exact form): every MFMA operand is fp16 (11-bit significand; bf16
// operands miss the 1e-3 state bar) with fp32 accumulation, except the diagonal 16 x 16 blocks of A_kk / A_qk, whose
// gated operands span e^{+-8|g|} and are taken as bf16 hi + lo pairs (3 MFMAs: hi.hi + hi.lo + lo.hi).  Off-diagonal
// blocks use the last row of the previous block as the reference point, so both gated operands are <= 1 (no overflow,
// only harmless underflow).  T is solved in fp32 (16 x 16 forward substitution + fp32 block products).  The state is
// fp32 throughout and is rounded to fp16 only as the B operand of W S / Qp S.
// Range note: fp16 operands hold |values| < 65504: the state, v and U must stay below that (the reference's relay has
// the same window, kda/mi350x/kda/kernel.py:113-128).  The diagonal blocks need |Gamma_i - Gamma_m| < 88 over 8
// tokens, i.e. a per-token log-decay above ~ -11 (always true for gate-in-kernel calls with lower_bound >= -11).
//
// Kernel 1, prologue: one workgroup (256 threads) per (chunk, head); writes the chunk's operands to the workspace.
// Kernel 2, walk: one workgroup (4 wave64) per (sequence, head); wave w owns value columns [32w, 32w + 32) and keeps
//   its 128 x 32 slice of S in MFMA accumulator registers for the whole sequence.  MFMA v_mfma_f32_16x16x32_f16:
//   A lane l holds row l%16, k-slots 8(l/16)..+7; B lane l holds column l%16, the same k-slots; C lane l holds rows
//   4(l/16)..+3 of column l%16.  Using the C layout of one product as the B operand of the next (no LDS round trip)
//   makes a lane's 8 k-slots the rows {4g..4g+3, 16+4g..16+4g+3} of a 32-row block (g = l/16); the workspace stores
//   W / Qp (channels) and Kd^T (tokens) in that permuted order so each A fragment is one 16-byte load.
#include <algorithm>
#include <numeric>
#include <vector>

#include "common.h"

namespace kda355 {
namespace {

constexpr int PF_THREADS = 256;
// workspace per (chunk, head), fp16 element offsets
constexpr int WS_W = 0;          // [64 tokens][128 channels], channels permuted within 32-blocks
constexpr int WS_QP = 8192;      // [64][128], channels permuted
constexpr int WS_KDT = 16384;    // [128 channels][64 tokens], tokens permuted within 32-blocks
constexpr int WS_UT = 24576;     // [128 values][64 tokens]
constexpr int WS_OIT = 32768;    // [128 values][64 tokens]
constexpr int WS_DEC_BYTES = 81920;  // fp32 [128] = e^{Gamma_c}
constexpr int64_t WS_BYTES = 82432;  // multiple of 256

constexpr uint32_t PLAN_MAGIC = 0x4b443535u;  // "KD55"
// table header words
enum { H_MAGIC = 0, H_N, H_T, H_NCHUNK, H_EVERY, H_OFF_CHUNK, H_OFF_CHAIN, H_OFF_SEQ, H_CKROWS, H_WORDS = 16 };

typedef _Float16 half_t;

__device__ __forceinline__ f32x4 mfma_f16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// position p (0..31) inside a 32-block for k-slot e (0..7) of lane group g
__device__ __forceinline__ int perm32(int g, int e) { return e < 4 ? 4 * g + e : 16 + 4 * g + (e - 4); }

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
    uint8_t* ws;
    int64_t qkv_rs, g_rs, beta_rs, out_rs;
    int64_t state_ss, state_slots, ck_ss, ck_slots;
    int N, H;
    float scale, lb;
    uint32_t flags;
    int ck_bf16;
};

// ------------------------------------------------------------------------------------------------ prologue
struct PrologueSmem {
    uint16_t q[64][128];    // raw bf16 rows (pad rows zero)
    uint16_t k[64][128];
    uint16_t v[64][128];
    float G[64][128];       // log-decay, then Gamma (inclusive cumsum) in place
    float rq[64], rk[64];   // 1 / max(|x|, 1e-6)
    float beta[64];
    float Akk[64][68];
    float Aqk[64][68];
    float T[64][68];
    float X[3][16][17];
};

template <bool RAW_GATE, bool RAW_BETA, bool NORM>
__global__ void __launch_bounds__(PF_THREADS) prologue_kernel(PfParams p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    PrologueSmem& sm = *reinterpret_cast<PrologueSmem*>(smem_raw);
    const int H = p.H;
    const int cg = blockIdx.x / H;
    const int h = blockIdx.x - cg * H;
    const int tid = threadIdx.x;
    const int wv = tid >> 6;
    const int lane = tid & 63;
    const int m = lane & 15;
    const int gq = lane >> 4;
    const int* chunk = p.tab + p.tab[H_OFF_CHUNK] + 2 * cg;
    const int t0 = chunk[0];
    const int L = chunk[1];

    // ---------------- load q, k, v (bf16), g, beta
    for (int i = tid; i < 64 * 16; i += PF_THREADS) {  // 16-byte pieces: row = i / 16, col8 = (i % 16) * 8
        const int r = i >> 4, c8 = (i & 15) * 8;
        u32x4 zq = {0, 0, 0, 0}, zk = zq, zv = zq;
        if (r < L) {
            const int64_t off = (int64_t)(t0 + r) * p.qkv_rs + (int64_t)h * D + c8;
            zq = *reinterpret_cast<const u32x4*>(p.q + off);
            zk = *reinterpret_cast<const u32x4*>(p.k + off);
            zv = *reinterpret_cast<const u32x4*>(p.v + off);
        }
        *reinterpret_cast<u32x4*>(&sm.q[r][c8]) = zq;
        *reinterpret_cast<u32x4*>(&sm.k[r][c8]) = zk;
        *reinterpret_cast<u32x4*>(&sm.v[r][c8]) = zv;
    }
    for (int i = tid; i < 64 * 32; i += PF_THREADS) {  // 4-float pieces
        const int r = i >> 5, c4 = (i & 31) * 4;
        f32x4 gv = {0.f, 0.f, 0.f, 0.f};
        if (r < L) {
            if (RAW_GATE) {
                const uint16_t* gb = reinterpret_cast<const uint16_t*>(p.g) + (int64_t)(t0 + r) * p.g_rs + h * D + c4;
                const u32x2 raw = *reinterpret_cast<const u32x2*>(gb);
                const float A = __expf(p.A_log[h]);
                const f32x4 db = *reinterpret_cast<const f32x4*>(p.dt_bias + h * D + c4);
                gv.x = p.lb * sigmoidf_(A * (bf2f(raw.x & 0xffffu) + db.x));
                gv.y = p.lb * sigmoidf_(A * (bf2f(raw.x >> 16) + db.y));
                gv.z = p.lb * sigmoidf_(A * (bf2f(raw.y & 0xffffu) + db.z));
                gv.w = p.lb * sigmoidf_(A * (bf2f(raw.y >> 16) + db.w));
            } else {
                gv = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p.g) + (int64_t)(t0 + r) * p.g_rs +
                                                     h * D + c4);
            }
        }
        *reinterpret_cast<f32x4*>(&sm.G[r][c4]) = gv;
    }
    if (tid < 64) {
        float b = 0.f;
        if (tid < L) {
            if (RAW_BETA)
                b = sigmoidf_(bf2f(reinterpret_cast<const uint16_t*>(p.beta)[(int64_t)(t0 + tid) * p.beta_rs + h]));
            else
                b = reinterpret_cast<const float*>(p.beta)[(int64_t)(t0 + tid) * p.beta_rs + h];
        }
        sm.beta[tid] = b;
    }
    // zero T (upper blocks stay zero)
    for (int i = tid; i < 64 * 68; i += PF_THREADS) (&sm.T[0][0])[i] = 0.f;
    __syncthreads();

    // ---------------- row norms (threads 0..127) and the gate cumsum (threads 128..255)
    if (tid < 128) {
        const int r = tid & 63;
        const uint16_t* row = (tid < 64) ? sm.q[r] : sm.k[r];
        float ss = 0.f;
        for (int c = 0; c < 128; c += 2) {
            const uint32_t w2 = *reinterpret_cast<const uint32_t*>(row + c);
            const float a = bf2f(w2 & 0xffffu), b = bf2f(w2 >> 16);
            ss += a * a + b * b;
        }
        float inv = 1.f;
        if (NORM) inv = 1.f / fmaxf(sqrtf(ss), 1e-6f);  // F.normalize (kda/mi350x/reference.py:59-60)
        if (tid < 64) sm.rq[r] = inv; else sm.rk[r] = inv;
    } else {
        const int c = tid - 128;
        float acc = 0.f;
        for (int r = 0; r < 64; ++r) {
            acc += sm.G[r][c];
            sm.G[r][c] = acc;
        }
    }
    __syncthreads();

    // ---------------- A_kk, A_qk: wave wv owns row block I = wv
    {
        const int I = wv;
        const int i = 16 * I + m;  // A-operand row of this lane
        const float rki = sm.rk[i], rqi = sm.rq[i];
        // diagonal block, reference row mr, bf16 hi/lo operands
        {
            const int mr = 16 * I + 7;
            f32x4 akk = {0.f, 0.f, 0.f, 0.f}, aqk = akk;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                bf16x8 ka_hi, ka_lo, qa_hi, qa_lo, kb_hi, kb_lo;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int c = 32 * s + 8 * gq + e;
                    const float gi = sm.G[i][c], gm = sm.G[mr][c];
                    const float fi = __expf(gi - gm), fj = __expf(gm - gi);  // row i as A, column i as B
                    const float kv = bf2f(sm.k[i][c]) * rki;
                    const float ka = kv * fi, qa = bf2f(sm.q[i][c]) * rqi * fi, kb = kv * fj;
                    const __bf16 kah = (__bf16)ka, qah = (__bf16)qa, kbh = (__bf16)kb;
                    ka_hi[e] = kah; ka_lo[e] = (__bf16)(ka - (float)kah);
                    qa_hi[e] = qah; qa_lo[e] = (__bf16)(qa - (float)qah);
                    kb_hi[e] = kbh; kb_lo[e] = (__bf16)(kb - (float)kbh);
                }
                akk = mfma_bf16(ka_hi, kb_hi, akk);
                akk = mfma_bf16(ka_hi, kb_lo, akk);
                akk = mfma_bf16(ka_lo, kb_hi, akk);
                aqk = mfma_bf16(qa_hi, kb_hi, aqk);
                aqk = mfma_bf16(qa_hi, kb_lo, aqk);
                aqk = mfma_bf16(qa_lo, kb_hi, aqk);
            }
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int row = 16 * I + 4 * gq + rr, col = 16 * I + m;
                sm.Akk[row][col] = (col < row) ? sm.beta[row] * akk[rr] : 0.f;
                sm.Aqk[row][col] = (col <= row) ? aqk[rr] : 0.f;
            }
        }
        // off-diagonal blocks (I, J < I), reference row r = 16 I - 1, fp16 operands <= 1
        if (I > 0) {
            const int r = 16 * I - 1;
            f16x8 kA[4], qA[4];
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int c = 32 * s + 8 * gq + e;
                    const float f = __expf(sm.G[i][c] - sm.G[r][c]);
                    kA[s][e] = (half_t)(bf2f(sm.k[i][c]) * rki * f);
                    qA[s][e] = (half_t)(bf2f(sm.q[i][c]) * rqi * f);
                }
            for (int J = 0; J < I; ++J) {
                const int j = 16 * J + m;  // B-operand column of this lane
                const float rkj = sm.rk[j];
                f32x4 akk = {0.f, 0.f, 0.f, 0.f}, aqk = akk;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    f16x8 kB;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int c = 32 * s + 8 * gq + e;
                        kB[e] = (half_t)(bf2f(sm.k[j][c]) * rkj * __expf(sm.G[r][c] - sm.G[j][c]));
                    }
                    akk = mfma_f16(kA[s], kB, akk);
                    aqk = mfma_f16(qA[s], kB, aqk);
                }
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int row = 16 * I + 4 * gq + rr, col = 16 * J + m;
                    sm.Akk[row][col] = sm.beta[row] * akk[rr];
                    sm.Aqk[row][col] = aqk[rr];
                }
            }
        }
        // zero the strictly-upper blocks of Aqk (read by the Qp / Oi products)
        for (int J = I + 1; J < 4; ++J)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) sm.Aqk[16 * I + 4 * gq + rr][16 * J + m] = 0.f;
    }
    __syncthreads();

    // ---------------- T = (I + A_kk)^-1: diagonal blocks by forward substitution (wave 0: lane = (block, column))
    if (wv == 0) {
        const int I = lane >> 4, j = lane & 15;
        float x[16];
#pragma unroll
        for (int ii = 0; ii < 16; ++ii) {
            float acc = 0.f;
#pragma unroll
            for (int mm = 0; mm < ii; ++mm) acc += sm.Akk[16 * I + ii][16 * I + mm] * x[mm];
            x[ii] = (ii < j) ? 0.f : ((ii == j) ? 1.f : -acc);
        }
#pragma unroll
        for (int ii = 0; ii < 16; ++ii) sm.T[16 * I + ii][16 * I + j] = x[ii];
    }
    __syncthreads();
    // off-diagonal blocks, by distance d = I - J: T_IJ = -T_II sum_{K=J}^{I-1} A_IK T_KJ
    for (int d = 1; d < 4; ++d) {
        const int cnt = 4 - d;
        for (int e = tid; e < cnt * 256; e += PF_THREADS) {
            const int b = e >> 8, ii = (e >> 4) & 15, jj = e & 15;
            const int I = d + b, J = b;
            float acc = 0.f;
            for (int K = J; K < I; ++K)
#pragma unroll
                for (int mm = 0; mm < 16; ++mm) acc += sm.Akk[16 * I + ii][16 * K + mm] * sm.T[16 * K + mm][16 * J + jj];
            sm.X[b][ii][jj] = acc;
        }
        __syncthreads();
        for (int e = tid; e < cnt * 256; e += PF_THREADS) {
            const int b = e >> 8, ii = (e >> 4) & 15, jj = e & 15;
            const int I = d + b, J = b;
            float acc = 0.f;
#pragma unroll
            for (int mm = 0; mm < 16; ++mm) acc += sm.T[16 * I + ii][16 * I + mm] * sm.X[b][mm][jj];
            sm.T[16 * I + ii][16 * J + jj] = -acc;
        }
        __syncthreads();
    }

    // ---------------- W = T diag(beta) K e^Gamma, U = T diag(beta) V: wave wv owns channels [32 wv, 32 wv + 32)
    uint8_t* ws = p.ws + ((int64_t)cg * H + h) * WS_BYTES;
    half_t* wsh = reinterpret_cast<half_t*>(ws);
    f32x4 Wacc[4][2], Uacc[4][2];
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            Wacc[it][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
            Uacc[it][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
    for (int s = 0; s < 2; ++s) {  // tokens 32 s .. 32 s + 31, natural k order: slot e of group gq = token 32 s + 8 gq + e
        f16x8 BW[2], BU[2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int c = 32 * wv + 16 * ct + m;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int j = 32 * s + 8 * gq + e;
                const float bj = sm.beta[j];
                BW[ct][e] = (half_t)(bj * bf2f(sm.k[j][c]) * sm.rk[j] * __expf(sm.G[j][c]));
                BU[ct][e] = (half_t)(bj * bf2f(sm.v[j][c]));
            }
        }
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            if (2 * s > it) continue;  // T[it block][tokens of k-step s] is zero
            f16x8 A;
            const float* trow = &sm.T[16 * it + m][32 * s + 8 * gq];
#pragma unroll
            for (int e = 0; e < 8; ++e) A[e] = (half_t)trow[e];
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                Wacc[it][ct] = mfma_f16(A, BW[ct], Wacc[it][ct]);
                Uacc[it][ct] = mfma_f16(A, BU[ct], Uacc[it][ct]);
            }
        }
    }
    // W -> workspace (channels permuted), U -> U^T (natural tokens)
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int pos = 16 * ct + m;  // natural position inside the 32-block of channels
            const int slot = pos < 16 ? 8 * (pos >> 2) + (pos & 3) : 8 * ((pos - 16) >> 2) + 4 + (pos & 3);
            const int cperm = 32 * wv + slot;
            const int c = 32 * wv + pos;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int row = 16 * it + 4 * gq + rr;
                wsh[WS_W + row * 128 + cperm] = (half_t)Wacc[it][ct][rr];
            }
            f16x4 u4;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) u4[rr] = (half_t)Uacc[it][ct][rr];
            *reinterpret_cast<f16x4*>(&wsh[WS_UT + c * 64 + 16 * it + 4 * gq]) = u4;
        }

    // ---------------- Qp = Q e^Gamma - A_qk W, Oi = A_qk U (B operands straight from the W / U accumulators)
    f32x4 Pacc[4][2], Oacc[4][2];
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            Pacc[it][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
            Oacc[it][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
    for (int s = 0; s < 2; ++s) {  // tokens of k-step s in permuted order: slot e of group gq = token 32 s + perm32(gq, e)
        f16x8 BW[2], BU[2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                BW[ct][rr] = (half_t)Wacc[2 * s][ct][rr];
                BW[ct][4 + rr] = (half_t)Wacc[2 * s + 1][ct][rr];
                BU[ct][rr] = (half_t)Uacc[2 * s][ct][rr];
                BU[ct][4 + rr] = (half_t)Uacc[2 * s + 1][ct][rr];
            }
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            if (2 * s > it) continue;
            f16x8 A;
            const float* arow = &sm.Aqk[16 * it + m][32 * s];
#pragma unroll
            for (int e = 0; e < 8; ++e) A[e] = (half_t)arow[perm32(gq, e)];
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                Pacc[it][ct] = mfma_f16(A, BW[ct], Pacc[it][ct]);
                Oacc[it][ct] = mfma_f16(A, BU[ct], Oacc[it][ct]);
            }
        }
    }
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int pos = 16 * ct + m;
            const int slot = pos < 16 ? 8 * (pos >> 2) + (pos & 3) : 8 * ((pos - 16) >> 2) + 4 + (pos & 3);
            const int cperm = 32 * wv + slot;
            const int c = 32 * wv + pos;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int row = 16 * it + 4 * gq + rr;
                const float qt = bf2f(sm.q[row][c]) * sm.rq[row] * __expf(sm.G[row][c]);
                wsh[WS_QP + row * 128 + cperm] = (half_t)(qt - Pacc[it][ct][rr]);
            }
            f16x4 o4;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) o4[rr] = (half_t)Oacc[it][ct][rr];
            *reinterpret_cast<f16x4*>(&wsh[WS_OIT + c * 64 + 16 * it + 4 * gq]) = o4;
        }

    // ---------------- Kd^T (tokens permuted) and the chunk decay
    for (int e = tid; e < 128 * 8; e += PF_THREADS) {
        const int c = e >> 3, grp8 = e & 7;  // 8 slots: block s = grp8 / 4, group g = grp8 % 4
        const int s = grp8 >> 2, g = grp8 & 3;
        const float gl = sm.G[63][c];
        f16x8 val;
#pragma unroll
        for (int ee = 0; ee < 8; ++ee) {
            const int t = 32 * s + perm32(g, ee);
            val[ee] = (half_t)(bf2f(sm.k[t][c]) * sm.rk[t] * __expf(gl - sm.G[t][c]));
        }
        *reinterpret_cast<f16x8*>(&wsh[WS_KDT + c * 64 + 8 * grp8]) = val;
    }
    if (tid < 128) reinterpret_cast<float*>(ws + WS_DEC_BYTES)[tid] = __expf(sm.G[63][tid]);
}

// ------------------------------------------------------------------------------------------------ walk
struct WalkSmem {
    half_t W[64][128];
    half_t Qp[64][128];
    half_t KdT[128][64];
};

__device__ __forceinline__ void store_state_rows(float* dst, const f32x4 (&S)[8][2], int wv, int gq, int m) {
    // dst: V-major [128 v][128 d]
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) {
        const int v = 32 * wv + 16 * vt + m;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(dst + v * 128 + 16 * dt + 4 * gq) = S[dt][vt];
    }
}
__device__ __forceinline__ void store_state_rows_bf16(uint16_t* dst, const f32x4 (&S)[8][2], int wv, int gq, int m) {
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) {
        const int v = 32 * wv + 16 * vt + m;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            u32x2 w;
            w.x = f2bf(S[dt][vt][0]) | (f2bf(S[dt][vt][1]) << 16);
            w.y = f2bf(S[dt][vt][2]) | (f2bf(S[dt][vt][3]) << 16);
            *reinterpret_cast<u32x2*>(dst + v * 128 + 16 * dt + 4 * gq) = w;
        }
    }
}

__global__ void __launch_bounds__(PF_THREADS) walk_kernel(PfParams p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    WalkSmem& sm = *reinterpret_cast<WalkSmem*>(smem_raw);
    const int H = p.H;
    const int ci = blockIdx.x / H;
    const int h = blockIdx.x - ci * H;
    const int tid = threadIdx.x;
    const int wv = tid >> 6;
    const int lane = tid & 63;
    const int m = lane & 15;
    const int gq = lane >> 4;
    const int* chain = p.tab + p.tab[H_OFF_CHAIN] + 4 * ci;
    const int n = chain[0], first = chain[1], nch = chain[2];
    const int* seqinfo = p.tab + p.tab[H_OFF_SEQ] + 2 * n;
    const int every = p.tab[H_EVERY];  // every-n checkpoint interval in chunks (0 = off)
    const bool pool = (p.flags & KDA355_PF_POOL) != 0;

    // ---- initial state
    f32x4 S[8][2];
    const float* src = nullptr;
    int64_t row = -1;
    if (pool) {
        row = p.state_idx[n];
        if (row >= 0 && row < p.state_slots && p.has_init[n]) src = p.state_pool + row * p.state_ss + (int64_t)h * D * D;
    } else if (p.init_state) {
        src = p.init_state + ((int64_t)n * H + h) * D * D;
    }
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) {
        const int v = 32 * wv + 16 * vt + m;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
            S[dt][vt] = src ? *reinterpret_cast<const f32x4*>(src + v * 128 + 16 * dt + 4 * gq) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // every-n checkpoint rows: row j = state before token j * every * 64 (j = 0: the initial state)
    const int ck_mode = (p.flags & KDA355_PF_CK_EVERY) ? 2 : ((p.flags & KDA355_PF_CK_SINGLE) ? 1 : 0);
    auto ck_store = [&](int64_t r) {
        if (r < 0 || r >= p.ck_slots) return;
        if (p.ck_bf16)
            store_state_rows_bf16(reinterpret_cast<uint16_t*>(p.ck_pool) + r * p.ck_ss + (int64_t)h * D * D, S, wv, gq, m);
        else
            store_state_rows(reinterpret_cast<float*>(p.ck_pool) + r * p.ck_ss + (int64_t)h * D * D, S, wv, gq, m);
    };
    if (ck_mode == 2 && every > 0 && nch > 0) ck_store(p.ck_idx[seqinfo[1]]);
    const int ck_single = (ck_mode == 1) ? seqinfo[0] : 0;  // chunk count after which the single checkpoint is taken

    const int* chunks = p.tab + p.tab[H_OFF_CHUNK];
    for (int cl = 0; cl < nch; ++cl) {
        const int cgl = first + cl;
        const int t0 = chunks[2 * cgl], L = chunks[2 * cgl + 1];
        const uint8_t* ws = p.ws + ((int64_t)cgl * H + h) * WS_BYTES;
        const half_t* wsh = reinterpret_cast<const half_t*>(ws);
        __syncthreads();  // previous chunk's LDS reads done
        {
            const u32x4* s4 = reinterpret_cast<const u32x4*>(wsh);  // W, Qp, KdT are the first 3 x 16 KiB
            u32x4* d4 = reinterpret_cast<u32x4*>(&sm.W[0][0]);
#pragma unroll
            for (int i = 0; i < 12; ++i) d4[i * PF_THREADS + tid] = s4[i * PF_THREADS + tid];
        }
        __syncthreads();
        // S -> fp16 B fragments (k = d in permuted order)
        f16x8 SB[4][2];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int vt = 0; vt < 2; ++vt)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    SB[s][vt][rr] = (half_t)S[2 * s][vt][rr];
                    SB[s][vt][4 + rr] = (half_t)S[2 * s + 1][vt][rr];
                }
        // V' = U - W S  (row tiles 0..3)
        f16x8 VB[2][2];
        f32x4 Vp[4][2];
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const f16x8 A = *reinterpret_cast<const f16x8*>(&sm.W[16 * it + m][32 * s + 8 * gq]);
                acc[0] = mfma_f16(A, SB[s][0], acc[0]);
                acc[1] = mfma_f16(A, SB[s][1], acc[1]);
            }
#pragma unroll
            for (int vt = 0; vt < 2; ++vt) {
                const int v = 32 * wv + 16 * vt + m;
                const f16x4 u4 = *reinterpret_cast<const f16x4*>(&wsh[WS_UT + v * 64 + 16 * it + 4 * gq]);
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) Vp[it][vt][rr] = (float)u4[rr] - acc[vt][rr];
            }
        }
        // O = scale (Qp S + Oi)  (row tiles 4..7)
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const f16x8 A = *reinterpret_cast<const f16x8*>(&sm.Qp[16 * it + m][32 * s + 8 * gq]);
                acc[0] = mfma_f16(A, SB[s][0], acc[0]);
                acc[1] = mfma_f16(A, SB[s][1], acc[1]);
            }
#pragma unroll
            for (int vt = 0; vt < 2; ++vt) {
                const int v = 32 * wv + 16 * vt + m;
                const f16x4 o4 = *reinterpret_cast<const f16x4*>(&wsh[WS_OIT + v * 64 + 16 * it + 4 * gq]);
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int i = 16 * it + 4 * gq + rr;
                    if (i < L)
                        p.out[(int64_t)(t0 + i) * p.out_rs + (int64_t)h * D + v] =
                            (uint16_t)f2bf(p.scale * (acc[vt][rr] + (float)o4[rr]));
                }
            }
        }
        // S <- diag(decay) S + Kd^T V'
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int vt = 0; vt < 2; ++vt)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    VB[s][vt][rr] = (half_t)Vp[2 * s][vt][rr];
                    VB[s][vt][4 + rr] = (half_t)Vp[2 * s + 1][vt][rr];
                }
        const float* dec = reinterpret_cast<const float*>(ws + WS_DEC_BYTES);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const f32x4 d4 = *reinterpret_cast<const f32x4*>(dec + 16 * dt + 4 * gq);
#pragma unroll
            for (int vt = 0; vt < 2; ++vt) {
                S[dt][vt][0] *= d4[0]; S[dt][vt][1] *= d4[1]; S[dt][vt][2] *= d4[2]; S[dt][vt][3] *= d4[3];
            }
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const f16x8 A = *reinterpret_cast<const f16x8*>(&sm.KdT[16 * dt + m][32 * s + 8 * gq]);
                S[dt][0] = mfma_f16(A, VB[s][0], S[dt][0]);
                S[dt][1] = mfma_f16(A, VB[s][1], S[dt][1]);
            }
        }
        // checkpoints at chunk boundaries
        if (ck_mode == 1 && cl + 1 == ck_single) ck_store(p.ck_idx[n]);
        if (ck_mode == 2 && every > 0 && (cl + 1) % every == 0 && cl + 1 < nch) ck_store(p.ck_idx[seqinfo[1] + (cl + 1) / every]);
    }
    // ---- final state
    if (pool) {
        if (row >= 0 && row < p.state_slots) store_state_rows(p.state_pool + row * p.state_ss + (int64_t)h * D * D, S, wv, gq, m);
    } else {
        store_state_rows(p.final_state + ((int64_t)n * H + h) * D * D, S, wv, gq, m);
    }
}

template <bool RG, bool RB, bool NM>
hipError_t launch_prologue(const PfParams& p, int nchunks, hipStream_t s) {
    const size_t smem = sizeof(PrologueSmem);
    static bool attr_set = false;  // idempotent; a race only repeats the call
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&prologue_kernel<RG, RB, NM>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL((prologue_kernel<RG, RB, NM>), dim3(nchunks * p.H), dim3(PF_THREADS), smem, s, p);
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
    int64_t nchunks = 0;
    for (int n = 0; n < N; ++n) nchunks += (cu[n + 1] - cu[n] + 63) / 64;
    const int64_t off_chunk = H_WORDS;
    const int64_t off_chain = off_chunk + 2 * nchunks;
    const int64_t off_seq = off_chain + 4 * (int64_t)N;
    const int64_t words = off_seq + 2 * (int64_t)N;
    plan->T = T;
    plan->N = N;
    plan->H = in->H;
    plan->num_chunks = (int32_t)nchunks;
    plan->num_chains = N;
    int maxc = 0;
    int64_t ckrows = 0;
    for (int n = 0; n < N; ++n) {
        const int c = (int)((cu[n + 1] - cu[n] + 63) / 64);
        maxc = std::max(maxc, c);
        if (every_chunks) ckrows += (c + every_chunks - 1) / every_chunks;
    }
    plan->max_chain_chunks = maxc;
    plan->table_words = words;
    plan->workspace_bytes = nchunks * (int64_t)in->H * WS_BYTES;
    plan->ck_rows = ckrows;
    plan->magic = PLAN_MAGIC;
    plan->flags = in->flags;
    plan->ck_every = in->ck_every;
    plan->reserved = 0;
    if (!tables) return 0;
    KDA_CHECK_ARG(capacity >= words, "prefill_plan: table capacity %lld < %lld words", (long long)capacity, (long long)words);
    int32_t* t = tables;
    std::fill(t, t + H_WORDS, 0);
    t[H_MAGIC] = (int32_t)PLAN_MAGIC;
    t[H_N] = N;
    t[H_T] = (int32_t)T;
    t[H_NCHUNK] = (int32_t)nchunks;
    t[H_EVERY] = every_chunks;
    t[H_OFF_CHUNK] = (int32_t)off_chunk;
    t[H_OFF_CHAIN] = (int32_t)off_chain;
    t[H_OFF_SEQ] = (int32_t)off_seq;
    t[H_CKROWS] = (int32_t)ckrows;
    std::vector<int> first(N);
    int64_t c = 0;
    int64_t ckstart = 0;
    for (int n = 0; n < N; ++n) {
        first[n] = (int)c;
        for (int64_t s0 = cu[n]; s0 < cu[n + 1]; s0 += 64, ++c) {
            t[off_chunk + 2 * c] = (int32_t)s0;
            t[off_chunk + 2 * c + 1] = (int32_t)std::min<int64_t>(64, cu[n + 1] - s0);
        }
        int ck_chunk = 0;
        if (in->ck_offsets) {
            const int32_t o = in->ck_offsets[n];
            // kda/mi350x/kda/prefill/main.cpp:110-118: offsets that are not positive multiples of 64 within the sequence
            // write nothing
            if (o > 0 && o % 64 == 0 && o <= cu[n + 1] - cu[n]) ck_chunk = o / 64;
        }
        t[off_seq + 2 * n] = ck_chunk;
        t[off_seq + 2 * n + 1] = (int32_t)ckstart;
        if (every_chunks) {
            const int cn = (int)((cu[n + 1] - cu[n] + 63) / 64);
            ckstart += (cn + every_chunks - 1) / every_chunks;
        }
    }
    // chains longest first (the walk's critical path starts earliest)
    std::vector<int> order(N);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return cu[a + 1] - cu[a] > cu[b + 1] - cu[b]; });
    for (int i = 0; i < N; ++i) {
        const int n = order[i];
        t[off_chain + 4 * i] = n;
        t[off_chain + 4 * i + 1] = first[n];
        t[off_chain + 4 * i + 2] = (int)((cu[n + 1] - cu[n] + 63) / 64);
        t[off_chain + 4 * i + 3] = (int32_t)cu[n];
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
    KDA_CHECK_ARG(pl->N == a->N && pl->T == a->T && pl->H == a->H,
                  "prefill: plan was made for another layout (N/T/H %d/%lld/%d vs %d/%lld/%d)", pl->N, (long long)pl->T,
                  pl->H, a->N, (long long)a->T, a->H);
    const uint32_t f = a->flags;
    KDA_CHECK_ARG(a->q && a->k && a->v && a->g && a->beta && a->out && a->tables, "prefill: a required pointer is null");
    KDA_CHECK_ARG(pl->num_chunks == 0 || a->workspace, "prefill: workspace is null");
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
    KDA_CHECK_ARG((f & KDA355_PF_RAW_GATE) ? (aligned(a->g, 8) && a->g_row_stride % 4 == 0)
                                           : (aligned(a->g, 16) && a->g_row_stride % 4 == 0),
                  "prefill: g rows misaligned");
    KDA_CHECK_ARG(aligned(a->out, 2), "prefill: out misaligned");
    KDA_CHECK_ARG(!pool || (aligned(a->state_pool, 16) && a->state_slot_stride % 4 == 0), "prefill: state pool misaligned");
    KDA_CHECK_ARG(pool || (aligned(a->final_state, 16) && (!a->initial_state || aligned(a->initial_state, 16))),
                  "prefill: states misaligned");
    KDA_CHECK_ARG(!a->ck_pool || (aligned(a->ck_pool, 16) && a->ck_slot_stride % 8 == 0), "prefill: ck pool misaligned");
    KDA_CHECK_ARG(aligned(a->workspace, 256), "prefill: workspace must be 256-byte aligned");
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
    p.ws = static_cast<uint8_t*>(a->workspace);
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
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipError_t e = hipSuccess;
    if (pl->num_chunks > 0) {
        const bool rg = f & KDA355_PF_RAW_GATE, rb = f & KDA355_PF_RAW_BETA, nm = f & KDA355_PF_NORMALIZE_QK;
        if (rg) {
            e = rb ? (nm ? launch_prologue<true, true, true>(p, pl->num_chunks, s) : launch_prologue<true, true, false>(p, pl->num_chunks, s))
                   : (nm ? launch_prologue<true, false, true>(p, pl->num_chunks, s) : launch_prologue<true, false, false>(p, pl->num_chunks, s));
        } else {
            e = rb ? (nm ? launch_prologue<false, true, true>(p, pl->num_chunks, s) : launch_prologue<false, true, false>(p, pl->num_chunks, s))
                   : (nm ? launch_prologue<false, false, true>(p, pl->num_chunks, s) : launch_prologue<false, false, false>(p, pl->num_chunks, s));
        }
        if (e != hipSuccess) {
            set_error("prefill: prologue launch failed: %s", hipGetErrorString(e));
            return KDA355_ELAUNCH;
        }
    }
    const size_t wsm = sizeof(WalkSmem);
    hipLaunchKernelGGL(walk_kernel, dim3(pl->num_chains * p.H), dim3(PF_THREADS), wsm, s, p);
    e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("prefill: walk launch failed: %s", hipGetErrorString(e));
        return KDA355_ELAUNCH;
    }
    return 0;
}
