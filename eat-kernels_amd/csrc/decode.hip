// Fused KDA decode / speculative verify on gfx950 (the vLLM-ROCm Kimi decode contract, kda/mi350x/kda/kernel.py:
// 212-216; semantics kda/mi350x/reference.py:104-181).
//
// One workgroup of 256 threads (4 wave64) per (sequence n, head h).  Per call:
//   * the head's 3 x 128 conv channels (q | k | v) of the window = 3 history taps of the bf16 conv cache followed by
//     the S input rows go to LDS with the conv weights; the width-4 causal conv + SiLU of all S tokens is computed up
//     front (it does not depend on the state), and the conv cache is committed: plain keeps the last 3 inputs, spec
//     keeps window[1:] (2 + S taps);
//   * the fp32 state (read row: idx[n] plain, idx[n, a-1] spec) is held in registers with the layout of the recurrent
//     kernel (lane: rows 16p + 4w + l/16, columns 4(l%16)..+3 and 64 + 4(l%16)..+3);
//   * per token: q, k <- x * rsqrt(sum x^2 + 1e-6) (q also * 128^-1/2, applied as the output scale), the gate
//     g = lb * sigmoid(exp(A_log[h]) * (gate + dt_bias)), beta = sigmoid(beta), the delta rule, then the gated RMSNorm
//     y = bf16(o) * rsqrt(mean(bf16(o)^2) + eps) * norm_weight * sigmoid(out_gate) on the 128 outputs of the head
//     (a cross-wave sum through LDS, double buffered per token); spec writes the state after token t to idx[n, t] > 0,
//     plain writes the final state back to idx[n].
// Slot rows <= 0 (and rows outside the pool) are padding (kda/mi350x/kda/decode/kda_v14_b.cu:1013-1042): a sequence
// whose read row or conv row is padding gets zero output rows and writes nothing; spec writes skip padding rows.
#include "common.h"

namespace kda355 {
namespace {

constexpr int DC_THREADS = 256;
constexpr int DC_MAX_S = 16;
constexpr int DC_CH = 3 * D;  // conv channels of one head: q | k | v

struct DecParams {
    const uint16_t* x;        // mixed_qkv [T, 3 * dim] bf16, row stride x_rs
    uint16_t* conv;           // conv_state [slots, taps, 3 * dim] bf16
    const float* cw;          // conv_weight [3, 4, dim] fp32
    const uint16_t* gate;     // [T, H, 128] bf16, row stride gate_rs
    const uint16_t* beta;     // [T, H] bf16 logits, row stride beta_rs
    const uint16_t* og;       // out_gate [T, dim] bf16, row stride og_rs
    const float* A_log;       // [H]
    const float* dt_bias;     // [H * 128]
    const float* nw;          // norm_weight [128]
    float* ssm;               // [slots, H, 128, 128] fp32, slot stride ssm_ss
    const int32_t* idx;       // [B] or [B, S]
    const int32_t* acc;       // [B] or null
    uint16_t* out;            // [T, dim] bf16, row stride out_rs
    int64_t x_rs, gate_rs, beta_rs, og_rs, out_rs;
    int64_t conv_ss, conv_ts, conv_slots, ssm_ss, ssm_slots;
    int B, S, H;
    float eps, lb, scale;
};

__device__ __forceinline__ bool slot_ok(int64_t r, int lo, int64_t n) { return r >= lo && r < n; }

template <bool SPEC>
__global__ void __launch_bounds__(DC_THREADS) decode_kernel(DecParams p) {
    // dynamic LDS: conv weights [4][384] fp32 | conv + SiLU outputs [S][384] fp32 | window [3 + S][384] bf16
    extern __shared__ __align__(16) float dsm[];
    float* sCw = dsm;
    float* sX = dsm + 4 * DC_CH;
    uint16_t* sWin = reinterpret_cast<uint16_t*>(dsm + (4 + p.S) * DC_CH);
    __shared__ float sO[2][D];                                        // head outputs of a token (double buffered)
    __shared__ float sRed[2][4];                                      // per-wave sums of squares

    const int n = blockIdx.x / p.H;
    const int h = blockIdx.x - n * p.H;
    const int tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63, grp = lane >> 4, j = lane & 15;
    const int S = p.S, H = p.H;
    const int dim = H * D;

    int a = 1;
    int64_t rd, cs;
    if (SPEC) {
        a = p.acc[n];
        a = a < 1 ? 1 : (a > S ? S : a);
        rd = p.idx[(int64_t)n * S + a - 1];
        cs = p.idx[(int64_t)n * S];
    } else {
        rd = p.idx[n];
        cs = rd;
    }
    const bool live = slot_ok(rd, 1, p.ssm_slots) && slot_ok(cs, 1, p.conv_slots);
    if (!live) {
        for (int t = 0; t < S; ++t) {
            uint32_t* o32 = reinterpret_cast<uint32_t*>(p.out + ((int64_t)n * S + t) * p.out_rs + h * D);
            if (tid < D / 2) o32[tid] = 0u;
        }
        return;
    }
    const int start = SPEC ? a - 1 : 0;

    // ---- state (issued first: the largest transfer), then the window and conv weights
    const int c0 = 4 * j;
    const float* src = p.ssm + rd * p.ssm_ss + (int64_t)h * D * D;
    f32x4 st[8][2];
#pragma unroll
    for (int pp = 0; pp < 8; ++pp) {
        const int row = pp * 16 + w * 4 + grp;
        st[pp][0] = *reinterpret_cast<const f32x4*>(src + row * D + c0);
        st[pp][1] = *reinterpret_cast<const f32x4*>(src + row * D + 64 + c0);
    }
    // ---- window (3 history taps + S inputs) and conv weights of this head's channels
    uint16_t* crow = p.conv + cs * p.conv_ss;
    for (int i = tid; i < (3 + S) * (DC_CH / 8); i += DC_THREADS) {  // 16-byte pieces: 8 channels
        const int r = i / (DC_CH / 8), c8 = (i % (DC_CH / 8)) * 8;
        const int grpc = c8 / D, ci = c8 % D;                        // q / k / v group, channel inside the head
        const int64_t col = (int64_t)grpc * dim + h * D + ci;
        const uint16_t* src = (r < 3) ? crow + (int64_t)(start + r) * p.conv_ts + col
                                      : p.x + ((int64_t)n * S + (r - 3)) * p.x_rs + col;
        *reinterpret_cast<u32x4*>(&sWin[r * DC_CH + c8]) = *reinterpret_cast<const u32x4*>(src);
    }
    for (int i = tid; i < 4 * DC_CH; i += DC_THREADS) {
        const int tap = i / DC_CH, c = i % DC_CH, grpc = c / D, ci = c % D;
        sCw[i] = p.cw[((int64_t)grpc * 4 + tap) * dim + h * D + ci];
    }
    __syncthreads();
    // ---- conv + SiLU for every token; conv cache commit
    for (int i = tid; i < S * DC_CH; i += DC_THREADS) {
        const int t = i / DC_CH, c = i % DC_CH;
        float acc = 0.f;
#pragma unroll
        for (int tap = 0; tap < 4; ++tap) acc += bf2f(sWin[(t + tap) * DC_CH + c]) * sCw[tap * DC_CH + c];
        sX[i] = acc * sigmoidf_(acc);
    }
    {
        // spec: taps [0, 2 + S) <- window[1 .. 3 + S);  plain: taps [0, 3) <- window[S .. S + 3)
        const int ntap = SPEC ? 2 + S : 3, first = SPEC ? 1 : S;
        for (int i = tid; i < ntap * (DC_CH / 8); i += DC_THREADS) {
            const int r = i / (DC_CH / 8), c8 = (i % (DC_CH / 8)) * 8;
            const int grpc = c8 / D, ci = c8 % D;
            *reinterpret_cast<u32x4*>(crow + (int64_t)r * p.conv_ts + (int64_t)grpc * dim + h * D + ci) =
                *reinterpret_cast<const u32x4*>(&sWin[(first + r) * DC_CH + c8]);
        }
    }
    const float A = __expf(p.A_log[h]);
    float db[8];
#pragma unroll
    for (int c = 0; c < 4; ++c) { db[c] = p.dt_bias[h * D + c0 + c]; db[4 + c] = p.dt_bias[h * D + 64 + c0 + c]; }
    __syncthreads();  // sX complete

    for (int t = 0; t < S; ++t) {
        const int64_t tok = (int64_t)n * S + t;
        const float* xq = sX + t * DC_CH;
        float kk[8], qq[8], dd[8], vv[8];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            qq[c] = xq[c0 + c]; qq[4 + c] = xq[64 + c0 + c];
            kk[c] = xq[D + c0 + c]; kk[4 + c] = xq[D + 64 + c0 + c];
        }
        {
            const uint16_t* gb = p.gate + tok * p.gate_rs + h * D;
            const u32x2 g0 = *reinterpret_cast<const u32x2*>(gb + c0);
            const u32x2 g1 = *reinterpret_cast<const u32x2*>(gb + 64 + c0);
            const float rg[8] = {bf2f(g0.x & 0xffffu), bf2f(g0.x >> 16), bf2f(g0.y & 0xffffu), bf2f(g0.y >> 16),
                                 bf2f(g1.x & 0xffffu), bf2f(g1.x >> 16), bf2f(g1.y & 0xffffu), bf2f(g1.y >> 16)};
#pragma unroll
            for (int c = 0; c < 8; ++c) dd[c] = __expf(p.lb * sigmoidf_(A * (rg[c] + db[c])));
        }
        const float bt = sigmoidf_(bf2f(p.beta[tok * p.beta_rs + h]));
        {  // x * rsqrt(sum x^2 + 1e-6)  (kda/mi350x/reference.py:159-160)
            float sk = 0.f, sq = 0.f;
#pragma unroll
            for (int c = 0; c < 8; ++c) { sk += kk[c] * kk[c]; sq += qq[c] * qq[c]; }
            sk = sum16(sk);
            sq = sum16(sq);
            const float ik = __frsqrt_rn(sk + 1e-6f), iq = __frsqrt_rn(sq + 1e-6f);
#pragma unroll
            for (int c = 0; c < 8; ++c) { kk[c] *= ik; qq[c] *= iq; }
        }
        float kq = 0.f;
#pragma unroll
        for (int c = 0; c < 8; ++c) kq += kk[c] * qq[c];
        kq = sum16(kq);
#pragma unroll
        for (int pp = 0; pp < 8; ++pp) vv[pp] = xq[2 * D + pp * 16 + w * 4 + grp];
        float ov[8];
#pragma unroll
        for (int pp = 0; pp < 8; ++pp) {
            st[pp][0].x *= dd[0]; st[pp][0].y *= dd[1]; st[pp][0].z *= dd[2]; st[pp][0].w *= dd[3];
            st[pp][1].x *= dd[4]; st[pp][1].y *= dd[5]; st[pp][1].z *= dd[6]; st[pp][1].w *= dd[7];
            float ak = st[pp][0].x * kk[0] + st[pp][0].y * kk[1] + st[pp][0].z * kk[2] + st[pp][0].w * kk[3] +
                       st[pp][1].x * kk[4] + st[pp][1].y * kk[5] + st[pp][1].z * kk[6] + st[pp][1].w * kk[7];
            float aq = st[pp][0].x * qq[0] + st[pp][0].y * qq[1] + st[pp][0].z * qq[2] + st[pp][0].w * qq[3] +
                       st[pp][1].x * qq[4] + st[pp][1].y * qq[5] + st[pp][1].z * qq[6] + st[pp][1].w * qq[7];
            ak = sum16(ak);
            aq = sum16(aq);
            const float u = bt * (vv[pp] - ak);
            ov[pp] = p.scale * (aq + u * kq);
            st[pp][0].x += u * kk[0]; st[pp][0].y += u * kk[1]; st[pp][0].z += u * kk[2]; st[pp][0].w += u * kk[3];
            st[pp][1].x += u * kk[4]; st[pp][1].y += u * kk[5]; st[pp][1].z += u * kk[6]; st[pp][1].w += u * kk[7];
        }
        if (j < 8) {  // lane j of each group holds row j * 16 + w * 4 + grp
            float o = ov[0];
#pragma unroll
            for (int pp = 1; pp < 8; ++pp) o = (j == pp) ? ov[pp] : o;
            sO[t & 1][j * 16 + w * 4 + grp] = o;
        }
        if (SPEC) {
            const int64_t wr = p.idx[(int64_t)n * S + t];
            if (slot_ok(wr, 1, p.ssm_slots)) {
                float* dst = p.ssm + wr * p.ssm_ss + (int64_t)h * D * D;
#pragma unroll
                for (int pp = 0; pp < 8; ++pp) {
                    const int row = pp * 16 + w * 4 + grp;
                    *reinterpret_cast<f32x4*>(dst + row * D + c0) = st[pp][0];
                    *reinterpret_cast<f32x4*>(dst + row * D + 64 + c0) = st[pp][1];
                }
            }
        }
        __syncthreads();
        // ---- gated RMSNorm over the head's 128 outputs (threads 0..127), y = bf16(o) rstd nw sigmoid(og)
        float ob = 0.f;
        if (tid < D) {
            ob = bf2f(f2bf(sO[t & 1][tid]));
            float ss = ob * ob;
            ss += __shfl_xor(ss, 32);
            ss = sum16(ss);
            ss += __shfl_xor(ss, 16);
            if (lane == 0) sRed[t & 1][w] = ss;
        }
        __syncthreads();
        if (tid < D) {
            const float rstd = __frsqrt_rn((sRed[t & 1][0] + sRed[t & 1][1]) * (1.f / D) + p.eps);
            const float g = bf2f(p.og[tok * p.og_rs + h * D + tid]);
            p.out[tok * p.out_rs + h * D + tid] = (uint16_t)f2bf(ob * rstd * p.nw[tid] * sigmoidf_(g));
        }
    }
    if (!SPEC) {
        float* dst = p.ssm + rd * p.ssm_ss + (int64_t)h * D * D;
#pragma unroll
        for (int pp = 0; pp < 8; ++pp) {
            const int row = pp * 16 + w * 4 + grp;
            *reinterpret_cast<f32x4*>(dst + row * D + c0) = st[pp][0];
            *reinterpret_cast<f32x4*>(dst + row * D + 64 + c0) = st[pp][1];
        }
    }
}

bool aligned(const void* q, size_t a) { return (reinterpret_cast<uintptr_t>(q) % a) == 0; }

}  // namespace
}  // namespace kda355

using namespace kda355;

extern "C" int kda355_decode_launch(const KdaDecodeArgs* a, kda355_stream_t stream) {
    KDA_CHECK_ARG(a != nullptr, "decode: null args");
    KDA_CHECK_ARG(a->B >= 0 && a->S >= 1 && a->S <= DC_MAX_S && a->H >= 1, "decode: B=%d S=%d H=%d (S <= %d)", a->B, a->S,
                  a->H, DC_MAX_S);
    if (a->B == 0) return 0;
    const bool spec = a->num_accepted != nullptr;
    KDA_CHECK_ARG(a->mixed_qkv && a->conv_state && a->conv_weight && a->gate && a->beta && a->out_gate && a->A_log &&
                      a->dt_bias && a->norm_weight && a->ssm_state && a->state_indices && a->out,
                  "decode: a required pointer is null");
    KDA_CHECK_ARG(a->conv_taps >= (spec ? 2 + a->S : 3), "decode: conv_state has %d taps, needs at least %d",
                  a->conv_taps, spec ? 2 + a->S : 3);
    KDA_CHECK_ARG(a->flags == 0, "decode: unknown flags 0x%x", a->flags);
    KDA_CHECK_ARG(a->conv_tap_stride >= 3 * a->H * D, "decode: conv_tap_stride %lld < 3 * H * 128",
                  (long long)a->conv_tap_stride);
    KDA_CHECK_ARG(aligned(a->out, 4) && a->out_row_stride % 2 == 0, "decode: out rows must be 4-byte aligned");
    KDA_CHECK_ARG(aligned(a->mixed_qkv, 16) && a->mixed_row_stride % 8 == 0, "decode: mixed_qkv rows must be 16-byte aligned");
    KDA_CHECK_ARG(aligned(a->conv_state, 16) && a->conv_slot_stride % 8 == 0 && a->conv_tap_stride % 8 == 0,
                  "decode: conv_state rows must be 16-byte aligned");
    KDA_CHECK_ARG(aligned(a->gate, 8) && a->gate_row_stride % 4 == 0, "decode: gate rows must be 8-byte aligned");
    KDA_CHECK_ARG(aligned(a->ssm_state, 16) && a->ssm_slot_stride % 4 == 0, "decode: ssm_state must be 16-byte aligned");
    KDA_CHECK_ARG((int64_t)a->B * a->H < (1ll << 31), "decode: grid too large");
    DecParams p;
    p.x = static_cast<const uint16_t*>(a->mixed_qkv);
    p.conv = static_cast<uint16_t*>(a->conv_state);
    p.cw = a->conv_weight;
    p.gate = static_cast<const uint16_t*>(a->gate);
    p.beta = static_cast<const uint16_t*>(a->beta);
    p.og = static_cast<const uint16_t*>(a->out_gate);
    p.A_log = a->A_log;
    p.dt_bias = a->dt_bias;
    p.nw = a->norm_weight;
    p.ssm = a->ssm_state;
    p.idx = a->state_indices;
    p.acc = a->num_accepted;
    p.out = static_cast<uint16_t*>(a->out);
    p.x_rs = a->mixed_row_stride;
    p.gate_rs = a->gate_row_stride;
    p.beta_rs = a->beta_row_stride;
    p.og_rs = a->out_gate_row_stride;
    p.out_rs = a->out_row_stride;
    p.conv_ss = a->conv_slot_stride;
    p.conv_ts = a->conv_tap_stride;
    p.conv_slots = a->conv_slots;
    p.ssm_ss = a->ssm_slot_stride;
    p.ssm_slots = a->ssm_slots;
    p.B = a->B;
    p.S = a->S;
    p.H = a->H;
    p.eps = a->norm_eps;
    p.lb = a->lower_bound;
    p.scale = 0.08838834764831845f;  // 128^-1/2: the reference scales the normalized q
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const size_t lds = (size_t)(4 + a->S) * DC_CH * sizeof(float) + (size_t)(3 + a->S) * DC_CH * sizeof(uint16_t);
    if (spec)
        hipLaunchKernelGGL(decode_kernel<true>, dim3(a->B * a->H), dim3(DC_THREADS), lds, s, p);
    else
        hipLaunchKernelGGL(decode_kernel<false>, dim3(a->B * a->H), dim3(DC_THREADS), lds, s, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("decode: launch failed: %s", hipGetErrorString(e));
        return KDA355_ELAUNCH;
    }
    return 0;
}
