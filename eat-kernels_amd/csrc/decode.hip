// Fused KDA decode / speculative verify on gfx950 (the vLLM-ROCm Kimi decode contract, kda/mi350x/kda/kernel.py:
// 212-216; semantics kda/mi350x/reference.py:104-181).
//
// One workgroup of 512 threads (8 wave64) per (sequence n, head h).  Per call:
//   * the head's 3 x 128 conv channels (q | k | v) of the window = 3 history taps of the bf16 conv cache followed by
//     the S input rows go to LDS with the conv weights; the width-4 causal conv + SiLU of all S tokens is computed up
//     front (it does not depend on the state), and the conv cache is committed: plain keeps the last 3 inputs, spec
//     keeps window[1:] (2 + S taps);
//   * the fp32 state (read row: idx[n] plain, idx[n, a-1] spec) is held in registers with the walker layout of
//     walk.h (lane: rows 16p + 2w + (l/32)%2, columns 4(l%32)..+3), streamed in and out with its cache policy;
//   * per token: q, k <- x * rsqrt(sum x^2 + 1e-6) (q also * 128^-1/2, applied as the output scale), the gate
//     g = lb * sigmoid(exp(A_log[h]) * (gate + dt_bias)), beta = sigmoid(beta), the delta rule, then the gated RMSNorm
//     y = bf16(o) * rsqrt(mean(bf16(o)^2) + eps) * norm_weight * sigmoid(out_gate) on the 128 outputs of the head
//     (bf16 outputs and per-half-wave sums of squares of every token kept in LDS, finished by all threads after the
//     walk behind one barrier); spec writes the state after token t to idx[n, t] > 0, plain writes the final state
//     back to idx[n].
// Slot rows <= 0 (and rows outside the pool) are padding (kda/mi350x/kda/decode/kda_v14_b.cu:1013-1042): a sequence
// whose read row or conv row is padding gets zero output rows and writes nothing; spec writes skip padding rows.
#include "walk.h"

namespace kda355 {
namespace {

constexpr int DC_THREADS = WK_THREADS;
constexpr int DC_MAX_S = 16;
constexpr int DC_CH = 3 * D;  // conv channels of one head: q | k | v
constexpr int64_t DC_SLICE_CUS = 256;  // a launch splits each state while the slices still fit one per CU (MI355X)
// Streaming stores from this many bytes of written state per launch.  Timed as the reference times decode (one graph
// replay after a 512 MiB cache flush, which is also what a layer's decode sees in a model of many layers: its pool rows
// were last touched a whole step earlier), streaming stores gain 1.5-3.5 % from 268 MB of writes up (d_glm16_b256
// 117.6 -> 115.8 us, s6_glm16_b64 105 -> 101.6 us, s8_h12_b64 102.7 -> 100.5 us) and lose below (s8_h12_b32, 201 MB:
// 56.6 -> 60.2 us; s8_h96_b1: 27.3 -> 33.1 us).
constexpr long long DC_STREAM_BYTES = 256ll << 20;

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
    int32_t* ws;              // sliced launches: counters [pairs] int32, then partial sums [pairs][VS][DC_MAX_S] fp32
    int B, S, H;
    float eps, lb, scale;
};
constexpr int DC_WS_PART = 256;  // byte offset of the partial sums (after DC_SLICE_CUS / 4 counters)

__device__ __forceinline__ bool slot_ok(int64_t r, int lo, int64_t n) { return r >= lo && r < n; }

// SINGLE: one token per sequence (plain decode), S = 1 known at compile time.
// PRE (several tokens, launches below the streaming size): the state-independent per-token operands are formed for
// every token before the walk, which shortens each token's step (the latency of a small launch is the tokens' steps
// in series); launches that stream more state than the MALL holds are bound by HBM, and there the extra phase and
// the higher occupancy its smaller register set allows measured 1-3 % slower, so they form them per token.
//
// NP < 8 (small launches, given a workspace): the state rows are split over VS = 8 / NP workgroups per (sequence,
// head), slice vs holding rows 16 NP vs .. 16 NP (vs + 1) - 1 (NP rows per lane), so a token's step is 8 / NP times
// shorter and 8 / NP times more CUs walk.  Every slice forms the conv and the q / k / gate operands of all 128 channels
// (the walk needs every key column).  Each slice writes bf16(o) of its rows to `out` and its per-token partial sums of
// squares to the workspace, then counts itself in the (sequence, head)'s counter (one vector atomic, no waiting); the
// slice that arrives last applies the gated RMSNorm to the 128 rows of every token, commits the conv cache (every
// slice has read the window by then) and sets the counter back to zero, so the workspace is all-zero counters again
// after every launch.  A slice cannot commit on its own: the other slices of its state may not have read the window
// yet.
// Streaming-store launches (more written state than the MALL holds) are held to fewer workgroups per CU: one for spec
// verify (2 waves per SIMD; s8_h96_b32 338 -> 322 us), two for single-token decode (4 waves per SIMD; the config-3
// shape 193 -> 189 us, one per CU measured slower); smaller launches keep the compiler's default.
template <bool SPEC, bool SINGLE, bool NT, int NP>
__global__ void __launch_bounds__(DC_THREADS)
    __attribute__((amdgpu_waves_per_eu(NT ? (SPEC ? 2 : 4) : 1, NT ? (SPEC ? 2 : 4) : 8))) decode_kernel(DecParams p) {
    constexpr bool PRE = !SINGLE && !NT;
    constexpr int VS = 8 / NP;  // slices per (sequence, head)
    // dynamic LDS: conv weights [4][384] fp32 | conv + SiLU outputs [S][384] fp32 | bf16-rounded outputs [S][128] fp32
    // | per-half-wave sums of squares [S][16] fp32 | gate factors exp(g) [S][128] fp32 | (k.q, beta) [S][2] fp32 |
    // window [3 + S][384] bf16
    extern __shared__ __align__(16) float dsm[];
    float* sCw = dsm;
    float* sX = sCw + 4 * DC_CH;
    float* sO = sX + p.S * DC_CH;
    float* sRed = sO + p.S * D;
    float* sDd = sRed + p.S * 16;
    float* sKB = sDd + p.S * D;
    uint16_t* sWin = reinterpret_cast<uint16_t*>(sKB + 2 * p.S);

    // (sequence, head) of this workgroup, kept in SGPRs: buffer descriptors built from them must be wave-uniform
    // values the compiler can see as such, or it wraps every buffer access in a waterfall loop
    const int task = xcd_task(blockIdx.x, gridDim.x);
    const int nh = __builtin_amdgcn_readfirstlane(task / VS);
    const int vs = __builtin_amdgcn_readfirstlane(task - nh * VS);
    const int n = __builtin_amdgcn_readfirstlane(nh / p.H);
    const int h = __builtin_amdgcn_readfirstlane(nh - n * p.H);
    const int row0 = 16 * NP * vs;  // the slice's first state row
    const int tid = threadIdx.x;
    const int S = SINGLE ? 1 : p.S, H = p.H;
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
        if (vs != 0) return;
        for (int t = 0; t < S; ++t) {
            uint32_t* o32 = reinterpret_cast<uint32_t*>(p.out + ((int64_t)n * S + t) * p.out_rs + h * D);
            if (tid < D / 2) o32[tid] = 0u;
        }
        return;
    }
    const int start = SPEC ? a - 1 : 0;
    const Walker wk(tid);
    const int c0 = 4 * wk.c;

    // ---- loads, in the order they are needed (vector memory completes in order): the window pieces and conv
    // weights, token 0's operands, then the state.  Nothing waits for the state until the first token's walk.
    uint16_t* crow = p.conv + cs * p.conv_ss;
    const int npieces = (3 + S) * (DC_CH / 8);  // 16-byte window pieces: 8 channels each, at most 2 per thread
    auto piece_src = [&](int i) {
        const int r = i / (DC_CH / 8), c8 = (i % (DC_CH / 8)) * 8;
        const int64_t col = (int64_t)(c8 / D) * dim + h * D + c8 % D;
        return (r < 3) ? crow + (int64_t)(start + r) * p.conv_ts + col : p.x + ((int64_t)n * S + (r - 3)) * p.x_rs + col;
    };
    // loads are unconditional (indices clamped): a load under a divergent branch makes the compiler wait for it
    // (vmcnt(0)) before the state loads are even issued
    const u32x4 wp0 = *reinterpret_cast<const u32x4*>(piece_src(min(tid, npieces - 1)));
    const u32x4 wp1 = *reinterpret_cast<const u32x4*>(piece_src(min(tid + DC_THREADS, npieces - 1)));
    // conv weights: 4 taps x 384 channels = 384 quads; quad i -> tap i / 96, channels 4 (i % 96) .. + 3
    const int cw_i = min(tid, DC_CH - 1);
    const int cw_tap = cw_i / (DC_CH / 4), cw_c = (cw_i % (DC_CH / 4)) * 4;
    const f32x4 cwq = *reinterpret_cast<const f32x4*>(p.cw + ((int64_t)(cw_c / D) * 4 + cw_tap) * dim + h * D + cw_c % D);
    // per-token scalars, lane t of each wave holding token t's (read back with readlane in the walk): the raw beta
    // and, in spec, the write row idx[n, t]
    const int lt = min(tid & 63, S - 1);
    const uint32_t beta_l = p.beta[((int64_t)n * S + lt) * p.beta_rs + h];
    const int32_t wr_l = SPEC ? p.idx[(int64_t)n * S + lt] : 0;
    auto load_gate = [&](int t) {
        return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                             row_rsrc(p.gate + ((int64_t)n * S + t) * p.gate_rs + h * D, D * 2), 8 * wk.c, 0, 0));
    };
    u32x2 g_next = PRE ? u32x2{0u, 0u} : load_gate(0);
    // PRE: the gate words of the tokens this wave forms before the walk (t = w, w + 8; clamped), channels 2 l, 2 l + 1
    const int l64 = tid & 63;
    uint32_t gw2[2] = {0u, 0u};
    f32x2 db2 = {0.f, 0.f};
    if (PRE) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
            gw2[j] = *reinterpret_cast<const uint32_t*>(p.gate + ((int64_t)n * S + min(wk.w + 8 * j, S - 1)) * p.gate_rs +
                                                        h * D + 2 * l64);
        db2 = *reinterpret_cast<const f32x2*>(p.dt_bias + h * D + 2 * l64);
    }
    // out_gate of the outputs this thread finishes after the walk: element i = tid + 512 k (token i / 128, row i % 128)
    constexpr int OG_PER = SINGLE ? 1 : (DC_MAX_S * D) / DC_THREADS;
    uint32_t ogv[OG_PER];
#pragma unroll
    for (int k = 0; k < OG_PER; ++k) {
        const int i = min(tid + k * DC_THREADS, S * D - 1);
        ogv[k] = __builtin_amdgcn_raw_buffer_load_b16(row_rsrc(p.og + ((int64_t)n * S + (i >> 7)) * p.og_rs + h * D, D * 2),
                                                      2 * (i & 127), 0, 0);
    }
    const float nw = p.nw[tid & (D - 1)];
    const float A = __expf(p.A_log[h]);
    const f32x4 db = *reinterpret_cast<const f32x4*>(p.dt_bias + h * D + c0);
    asm volatile("" ::: "memory");  // keep the loads above ahead of the state loads (completion is in issue order)
    f32x4 st[NP];
    const int64_t slice = (int64_t)h * D * D + (int64_t)row0 * D;  // the slice's first element in a pool row
    load_state<NP>(wk, p.ssm + rd * p.ssm_ss + slice, st);

    // unconditional: threads past the end rewrite the last piece / quad with the same data
    *reinterpret_cast<u32x4*>(&sWin[min(tid, npieces - 1) * 8]) = wp0;
    *reinterpret_cast<u32x4*>(&sWin[min(tid + DC_THREADS, npieces - 1) * 8]) = wp1;
    *reinterpret_cast<f32x4*>(&sCw[cw_tap * DC_CH + cw_c]) = cwq;
    // nw * sigmoid(out_gate) of this thread's outputs, formed now: these loads are older than the state loads, and
    // consuming them here keeps the epilogue from waiting on the state stores
    float ogw[OG_PER];
#pragma unroll
    for (int k = 0; k < OG_PER; ++k) ogw[k] = nw * sigmoidf_(bf2f(ogv[k]));
    const float dbA[4] = {A * db.x, A * db.y, A * db.z, A * db.w};  // gate = lb sigmoid(A gate + A dt_bias)
    lds_barrier();
    // ---- conv + SiLU for every token; conv cache commit
#pragma unroll 1
    for (int i = tid; i < S * DC_CH; i += DC_THREADS) {
        const int t = i / DC_CH, c = i % DC_CH;
        float acc = 0.f;
#pragma unroll
        for (int tap = 0; tap < 4; ++tap) acc += bf2f(sWin[(t + tap) * DC_CH + c]) * sCw[tap * DC_CH + c];
        sX[i] = acc * sigmoidf_(acc);
    }
    // conv cache commit from the window in LDS; spec: taps [0, 2 + S) <- window[1 .. 3 + S);  plain: taps [0, 3) <-
    // window[S .. S + 3)
    auto conv_commit = [&]() {
        const int ntap = SPEC ? 2 + S : 3, first = SPEC ? 1 : S;
#pragma unroll 1
        for (int i = tid; i < ntap * (DC_CH / 8); i += DC_THREADS) {
            const int r = i / (DC_CH / 8), c8 = (i % (DC_CH / 8)) * 8;
            const int grpc = c8 / D, ci = c8 % D;
            *reinterpret_cast<u32x4*>(crow + (int64_t)r * p.conv_ts + (int64_t)grpc * dim + h * D + ci) =
                *reinterpret_cast<const u32x4*>(&sWin[(first + r) * DC_CH + c8]);
        }
    };
    if constexpr (NP == 8) conv_commit();  // (a sliced launch commits in its last slice, after every slice has read
                                           // the window)
    lds_barrier();  // sX complete
    if (PRE) {
        // the per-token operands that do not depend on the state, formed before the walk (wave w takes tokens w and
        // w + 8): q and k normalized in place in sX, exp(g) of the 128 channels, k . q and sigmoid(beta)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int t = wk.w + 8 * j;
            if (t < S) {  // wave-uniform
                float* xq = sX + t * DC_CH;
                f32x2 qx = *reinterpret_cast<const f32x2*>(xq + 2 * l64);
                f32x2 kx = *reinterpret_cast<const f32x2*>(xq + D + 2 * l64);
                const float rq = __frsqrt_rn(sum64(qx.x * qx.x + qx.y * qx.y) + 1e-6f);
                const float rk = __frsqrt_rn(sum64(kx.x * kx.x + kx.y * kx.y) + 1e-6f);
                qx *= rq;
                kx *= rk;
                *reinterpret_cast<f32x2*>(xq + 2 * l64) = qx;
                *reinterpret_cast<f32x2*>(xq + D + 2 * l64) = kx;
                const float kq = sum64(qx.x * kx.x + qx.y * kx.y);
                const f32x2 dd = {__expf(p.lb * sigmoidf_(A * bf2f(gw2[j] & 0xffffu) + A * db2.x)),
                                  __expf(p.lb * sigmoidf_(A * bf2f(gw2[j] >> 16) + A * db2.y))};
                *reinterpret_cast<f32x2*>(sDd + t * D + 2 * l64) = dd;
                if (l64 == 0) {
                    sKB[2 * t] = kq;
                    sKB[2 * t + 1] = sigmoidf_(bf2f(__builtin_amdgcn_readlane(beta_l, t) & 0xffffu));
                }
            }
        }
        lds_barrier();
    }
    if (!SINGLE) state_ready(st);
    // v of the slice row this lane broadcasts (lanes with c % 8 >= NP repeat the last one)
    const int vrow = row0 + 16 * min(wk.c & 7, NP - 1) + 2 * wk.w + wk.half;

    for (int t = 0; t < S; ++t) {
        const float* xq = sX + t * DC_CH;
        const f32x4 q4 = *reinterpret_cast<const f32x4*>(xq + c0);
        const f32x4 k4 = *reinterpret_cast<const f32x4*>(xq + D + c0);
        float qq[4] = {q4.x, q4.y, q4.z, q4.w};
        float kk[4] = {k4.x, k4.y, k4.z, k4.w};
        float dd[4], o;
        if (!PRE) {
            const u32x2 gcur = g_next;
            g_next = load_gate(min(t + 1, S - 1));  // unconditional, issued before this token's state stores
            const float rg[4] = {bf2f(gcur.x & 0xffffu), bf2f(gcur.x >> 16), bf2f(gcur.y & 0xffffu), bf2f(gcur.y >> 16)};
#pragma unroll
            for (int c = 0; c < 4; ++c) dd[c] = __expf(p.lb * sigmoidf_(A * rg[c] + dbA[c]));
            rsqrt_norm4(kk);  // x * rsqrt(sum x^2 + 1e-6)  (kda/mi350x/reference.py:159-160)
            rsqrt_norm4(qq);
            const float bt = sigmoidf_(bf2f(__builtin_amdgcn_readlane(beta_l, t) & 0xffffu));
            o = walk_token<NP>(st, kk, qq, dd, xq[2 * D + vrow], bt, p.scale, wk.c);
        } else {
            const f32x4 d4 = *reinterpret_cast<const f32x4*>(sDd + t * D + c0);
            dd[0] = d4.x; dd[1] = d4.y; dd[2] = d4.z; dd[3] = d4.w;
            o = walk_token_kq<NP>(st, kk, qq, dd, xq[2 * D + vrow], sKB[2 * t + 1], sKB[2 * t], p.scale, wk.c);
        }
        if constexpr (NP == 8) {
            // bf16(o) of the lane's row and the half wave's sum of squares (lanes c < 8 hold the half's 8 rows)
            const float ob = bf2f(f2bf(o));
            const float ss = sum32(wk.c < 8 ? ob * ob : 0.f);
            if (wk.c < 8) sO[t * D + wk.row(wk.c)] = ob;
            if (wk.c == 0) sRed[t * 16 + 2 * wk.w + wk.half] = ss;
        } else {  // bf16(o) of the slice's rows straight to `out` and the half wave's sum of squares; the last slice
                  // finishes them
            const uint32_t o16 = f2bf(o);
            if (wk.c < NP)
                __hip_atomic_store(p.out + ((int64_t)n * S + t) * p.out_rs + h * D + row0 + wk.row(wk.c), (uint16_t)o16,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float ob = bf2f(o16);
            const float ss = sum32(wk.c < NP ? ob * ob : 0.f);
            if (wk.c == 0) sRed[t * 16 + 2 * wk.w + wk.half] = ss;
        }
        if (SPEC) {
            const int64_t wr = __builtin_amdgcn_readlane(wr_l, t);
            const bool ok = slot_ok(wr, 1, p.ssm_slots);
            store_state<NT, NP>(wk, p.ssm + (ok ? wr : 0) * p.ssm_ss + slice, st, ok);
        }
    }
    if (!SPEC) store_state<NT, NP>(wk, p.ssm + rd * p.ssm_ss + slice, st);
    if constexpr (NP < 8) {
        // The rows and sums the slices exchange are written and read with device-scope (coherent) accesses: the
        // slices of one head may sit on different XCDs, whose L2s are not coherent with each other, and a full L2
        // write-back (a device-scope fence) costs the whole launch several microseconds after a cache flush.
        float* part = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(p.ws) + DC_WS_PART);
        lds_barrier();  // sRed complete
        if (tid < S) {
            const f32x4* r4 = reinterpret_cast<const f32x4*>(sRed + tid * 16);
            const f32x4 s4 = (r4[0] + r4[1]) + (r4[2] + r4[3]);
            __hip_atomic_store(part + ((int64_t)nh * VS + vs) * DC_MAX_S + tid, (s4.x + s4.y) + (s4.z + s4.w),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();  // every thread's coherent stores have completed (the barrier waits for them)
        int* s_arrive = reinterpret_cast<int*>(sKB);  // (k . q, beta) are dead after the walk
        if (tid == 0) s_arrive[0] = __hip_atomic_fetch_add(p.ws + nh, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (s_arrive[0] != VS - 1) return;  // workgroup-uniform: the last slice to arrive finishes the head
#pragma unroll
        for (int k = 0; k < OG_PER; ++k) {
            const int i = tid + k * DC_THREADS;
            if (i < S * D) {
                const int t = i >> 7;
                float ss = 0.f;
#pragma unroll
                for (int j = 0; j < VS; ++j)
                    ss += __hip_atomic_load(part + ((int64_t)nh * VS + j) * DC_MAX_S + t, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
                const float rstd = __frsqrt_rn(ss * (1.f / D) + p.eps);
                uint16_t* o = p.out + ((int64_t)n * S + t) * p.out_rs + h * D + (i & 127);
                const uint16_t x = __hip_atomic_load(o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                *o = (uint16_t)f2bf(bf2f(x) * rstd * ogw[k]);
            }
        }
        conv_commit();
        if (tid == 0) p.ws[nh] = 0;  // the next launch starts from a zero counter
        return;
    }
    lds_barrier();
    // ---- gated RMSNorm of every token's 128 outputs: y = bf16(o) rsqrt(mean(bf16(o)^2) + eps) nw sigmoid(og)
#pragma unroll
    for (int k = 0; k < OG_PER; ++k) {
        const int i = tid + k * DC_THREADS;
        if (i < S * D) {
            const int t = i >> 7;
            const f32x4* r4 = reinterpret_cast<const f32x4*>(sRed + t * 16);
            const f32x4 s4 = (r4[0] + r4[1]) + (r4[2] + r4[3]);
            const float rstd = __frsqrt_rn((s4.x + s4.y + s4.z + s4.w) * (1.f / D) + p.eps);
            const float y = sO[i] * rstd * ogw[k];
            __builtin_amdgcn_raw_buffer_store_b16((unsigned short)f2bf(y),
                                                  row_rsrc(p.out + ((int64_t)n * S + t) * p.out_rs + h * D, D * 2),
                                                  2 * (i & 127), 0, 0);
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
    KDA_CHECK_ARG(aligned(a->conv_weight, 16) && aligned(a->dt_bias, 16), "decode: conv_weight and dt_bias must be 16-byte aligned");
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
    p.ws = static_cast<int32_t*>(a->workspace);
    p.scale = 0.08838834764831845f;  // 128^-1/2: the reference scales the normalized q
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const size_t lds = ((size_t)(4 + a->S) * DC_CH + (size_t)a->S * (2 * D + 18)) * sizeof(float) +
                       (size_t)(3 + a->S) * DC_CH * sizeof(uint16_t);
    const bool nt = (long long)a->B * (spec ? a->S : 1) * a->H * D * D * 4 >= DC_STREAM_BYTES;
    // Small launches split each state over 4 workgroups (32 rows each) while the slices fit one per CU, so that more
    // CUs walk and each token's step is shorter; the last slice of each (sequence, head) finishes its rows, which needs
    // the caller's workspace (without one, whole states).  (Halves of 64 rows for launches of up to 128 pairs measured
    // no faster than whole states: s8_h96_b1 27.5 against 27.1 us.)
    const int64_t pairs = (int64_t)a->B * a->H;
    const int np = (a->workspace && !nt && 4 * pairs <= DC_SLICE_CUS) ? 2 : 8;
    void (*kernel)(DecParams) =
        np == 2 ? (spec ? decode_kernel<true, false, false, 2>
                        : a->S == 1 ? decode_kernel<false, true, false, 2> : decode_kernel<false, false, false, 2>)
        : spec ? (nt ? decode_kernel<true, false, true, 8> : decode_kernel<true, false, false, 8>)
        : a->S == 1 ? (nt ? decode_kernel<false, true, true, 8> : decode_kernel<false, true, false, 8>)
                    : (nt ? decode_kernel<false, false, true, 8> : decode_kernel<false, false, false, 8>);
    hipLaunchKernelGGL(kernel, dim3(a->B * a->H * (8 / np)), dim3(DC_THREADS), lds, s, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("decode: launch failed: %s", hipGetErrorString(e));
        return KDA355_ELAUNCH;
    }
    return 0;
}
