// Recurrent KDA decode / speculative verify on gfx950, and the commit of an accepted draft length.
//
// The step is a bandwidth-bound read-modify-write of the fp32 128 x 128 state of each (sequence, head): 64 KiB read,
// 64 KiB written per stored state.  One workgroup of 512 threads (8 wave64) owns one (sequence, head) and walks its
// tokens with the state in registers (walk.h: row layout, cache policy, 32-lane row reductions);
// o_t = scale * (S' q + u (k . q)) with S' the decayed state before the rank-1 update -- the two reductions are
// independent, so they are issued together (algebraically the reference's o = scale * S_new q).
// Semantics: kda/mi350x/reference.py:155-171 (recurrent core), slot rules kda/mi350x/kda/decode/kda_v14_b.cu:1013-1042
// (padding slot 0 and out-of-range rows are never read or written; such a sequence's output rows are zero).
#include "walk.h"

namespace kda355 {
namespace {

constexpr int REC_THREADS = WK_THREADS;

struct RecParams {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const void* g;
    const void* beta;
    const float* A_log;
    const float* dt_bias;
    float* read_pool;
    float* write_pool;
    const int32_t* read_idx;
    const int32_t* num_accepted;
    const int32_t* write_idx;
    uint16_t* out;
    int64_t qkv_rs, g_rs, beta_rs, out_rs;
    int64_t read_ss, read_slots, write_ss, write_slots;
    int B, S, H, read_idx_stride;
    int read_min, write_min;  // smallest valid row of each pool (1 when row 0 is the reserved padding slot)
    float scale, lb;
};

__device__ __forceinline__ bool row_ok(int64_t r, int64_t lo, int64_t slots) { return r >= lo && r < slots; }

// MODE: REC_SINGLE one token per sequence (plain decode, S = 1 known at compile time), REC_MULTI several tokens with
// the final state written back, REC_PER_TOKEN the state after every token written (spec verify).
enum { REC_SINGLE = 0, REC_MULTI = 1, REC_PER_TOKEN_MODE = 2 };

// The streaming-store instantiations (launches that write more state than the MALL holds) are held to 2 waves per
// SIMD, one workgroup per CU: an HBM-bound stream of state rows runs faster with fewer workgroups in flight per CU
// (config 3 179 -> 173 us, spec verify H = 64 234 -> 226 us); smaller launches keep the compiler's default.
template <bool RAW_GATE, bool RAW_BETA, bool NORM, int MODE, bool NT>
__global__ void __launch_bounds__(REC_THREADS) __attribute__((amdgpu_waves_per_eu(NT ? 2 : 1, NT ? 2 : 8)))
recurrent_kernel(RecParams p) {
    constexpr bool PER_TOKEN = MODE == REC_PER_TOKEN_MODE;
    // (sequence, head) of this workgroup, kept in SGPRs: buffer descriptors built from them must be wave-uniform
    // values the compiler can see as such, or it wraps every buffer access in a waterfall loop
    const int task = xcd_task(blockIdx.x, gridDim.x);
    const int n = __builtin_amdgcn_readfirstlane(task / p.H);
    const int h = __builtin_amdgcn_readfirstlane(task - n * p.H);
    const int tid = threadIdx.x;
    const int S = MODE == REC_SINGLE ? 1 : p.S;

    int a = 1;
    if (p.num_accepted) {
        a = p.num_accepted[n];
        a = a < 1 ? 1 : (a > S ? S : a);
    }
    const int64_t rd = p.read_idx[(int64_t)n * p.read_idx_stride + (p.num_accepted ? a - 1 : 0)];
    const bool live = row_ok(rd, p.read_min, p.read_slots);

    if (!live) {  // padding sequence: zero output rows, no state traffic
        for (int t = 0; t < S; ++t) {
            const int64_t tok = (int64_t)n * S + t;
            if (tid < D / 2) {
                uint32_t* o32 = reinterpret_cast<uint32_t*>(p.out + tok * p.out_rs + h * D);
                o32[tid] = 0u;
            }
        }
        return;
    }

    // Per-token operands of this head, raw (converted at use).  Token t + 1's are loaded before token t's state
    // stores and token 0's before the state loads: vector memory completes in order, so an operand never waits
    // behind a state transfer issued after it.
    const Walker wk(tid);
    // raw beta and (per-token writes) the write row of token t, held by lane t of each wave, read back with readlane
    const int lt = min(tid & 63, S - 1);
    const uint32_t beta_l = RAW_BETA ? (uint32_t)reinterpret_cast<const uint16_t*>(p.beta)[((int64_t)n * S + lt) * p.beta_rs + h]
                                     : __float_as_uint(reinterpret_cast<const float*>(p.beta)[((int64_t)n * S + lt) * p.beta_rs + h]);
    const int32_t wr_l = PER_TOKEN ? p.write_idx[(int64_t)n * S + lt] : 0;
    struct Ops { u32x2 k, q, g2; f32x4 g4; uint32_t v; };
    auto load_ops = [&](int t) {
        Ops o;
        const int64_t tok = (int64_t)n * S + t;
        const int64_t ro = tok * p.qkv_rs + h * D;
        o.k = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(row_rsrc(p.k + ro, D * 2), 8 * wk.c, 0, 0));
        o.q = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(row_rsrc(p.q + ro, D * 2), 8 * wk.c, 0, 0));
        o.v = __builtin_amdgcn_raw_buffer_load_b16(row_rsrc(p.v + ro, D * 2), 2 * v_src_row(wk), 0, 0);
        if (RAW_GATE)
            o.g2 = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                row_rsrc(reinterpret_cast<const uint16_t*>(p.g) + tok * p.g_rs + h * D, D * 2), 8 * wk.c, 0, 0));
        else
            o.g4 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                row_rsrc(reinterpret_cast<const float*>(p.g) + tok * p.g_rs + h * D, D * 4), 16 * wk.c, 0, 0));
        return o;
    };
    Ops op = load_ops(0);
    // ---- state: 8 rows x 4 columns per lane
    f32x4 st[8];
    load_state(wk, p.read_pool + rd * p.read_ss + (int64_t)h * D * D, st);
    float A = 0.f, db[4] = {0.f, 0.f, 0.f, 0.f};
    if (RAW_GATE) {
        A = __expf(p.A_log[h]);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(p.dt_bias + h * D + 4 * wk.c);
        db[0] = d4.x; db[1] = d4.y; db[2] = d4.z; db[3] = d4.w;
    }

    if (MODE != REC_SINGLE) state_ready(st);
    for (int t = 0; t < S; ++t) {
        const int64_t tok = (int64_t)n * S + t;
        const Ops cur = op;
        if (MODE != REC_SINGLE) op = load_ops(min(t + 1, S - 1));  // unconditional, issued before this token's stores
        const uint32_t braw = __builtin_amdgcn_readlane(beta_l, t);
        const float bt = RAW_BETA ? sigmoidf_(bf2f(braw & 0xffffu)) : __uint_as_float(braw);
        float kk[4] = {bf2f(cur.k.x & 0xffffu), bf2f(cur.k.x >> 16), bf2f(cur.k.y & 0xffffu), bf2f(cur.k.y >> 16)};
        float qq[4] = {bf2f(cur.q.x & 0xffffu), bf2f(cur.q.x >> 16), bf2f(cur.q.y & 0xffffu), bf2f(cur.q.y >> 16)};
        float dd[4];
        if (RAW_GATE) {
            const float rg[4] = {bf2f(cur.g2.x & 0xffffu), bf2f(cur.g2.x >> 16), bf2f(cur.g2.y & 0xffffu),
                                 bf2f(cur.g2.y >> 16)};
#pragma unroll
            for (int c = 0; c < 4; ++c) dd[c] = __expf(p.lb * sigmoidf_(A * (rg[c] + db[c])));
        } else {
            dd[0] = __expf(cur.g4.x); dd[1] = __expf(cur.g4.y); dd[2] = __expf(cur.g4.z); dd[3] = __expf(cur.g4.w);
        }
        if (NORM) {  // x * rsqrt(sum x^2 + 1e-6)  (kda/mi350x/reference.py:159-160)
            rsqrt_norm4(kk);
            rsqrt_norm4(qq);
        }
        const float o = walk_token(st, kk, qq, dd, bf2f(cur.v), bt, p.scale, wk.c);
        // output: lane c < 8 of each half wave writes row 16 c + 2 w + half
        if (wk.c < 8)
            __builtin_amdgcn_raw_buffer_store_b16((unsigned short)f2bf(o), row_rsrc(p.out + tok * p.out_rs + h * D, D * 2),
                                                  2 * wk.row(wk.c), 0, 0);
        if (PER_TOKEN) {
            const int64_t wr = __builtin_amdgcn_readlane(wr_l, t);
            const bool ok = row_ok(wr, p.write_min, p.write_slots);
            store_state<NT>(wk, p.write_pool + (ok ? wr : 0) * p.write_ss + (int64_t)h * D * D, st, ok);
        }
    }
    if (!PER_TOKEN) store_state<NT>(wk, p.read_pool + rd * p.read_ss + (int64_t)h * D * D, st);
}

// Copy one (sequence, head) state: scratch[scratch_idx[n, a-1]] -> pool[pool_idx[n]].
template <bool NT>
__global__ void __launch_bounds__(WK_THREADS) spec_commit_kernel(KdaSpecCommitArgs a, bool slot0) {
    const int task = xcd_task(blockIdx.x, gridDim.x);
    const int n = __builtin_amdgcn_readfirstlane(task / a.H);
    const int h = __builtin_amdgcn_readfirstlane(task - n * a.H);
    int acc = a.num_accepted[n];
    acc = acc < 1 ? 1 : (acc > a.S ? a.S : acc);
    const int64_t sr = a.scratch_idx[(int64_t)n * a.S + acc - 1];
    const int64_t pr = a.pool_idx[n];
    if (sr < 0 || sr >= a.scratch_slots || pr < (slot0 ? 1 : 0) || pr >= a.pool_slots) return;
    const Walker wk(threadIdx.x);
    f32x4 buf[8];
    load_state(wk, a.scratch + sr * a.scratch_slot_stride + (int64_t)h * D * D, buf);
    store_state<NT>(wk, a.pool + pr * a.pool_slot_stride + (int64_t)h * D * D, buf);
}

// streaming stores when the launch writes more state than the MALL holds (WK_STREAM_BYTES)
template <bool RG, bool RB, bool NM, int MODE>
hipError_t launch_rec(const RecParams& p, hipStream_t s) {
    const long long written = (long long)p.B * (MODE == REC_PER_TOKEN_MODE ? p.S : 1) * p.H * D * D * 4;
    if (written > WK_STREAM_BYTES)
        hipLaunchKernelGGL((recurrent_kernel<RG, RB, NM, MODE, true>), dim3(p.B * p.H), dim3(REC_THREADS), 0, s, p);
    else
        hipLaunchKernelGGL((recurrent_kernel<RG, RB, NM, MODE, false>), dim3(p.B * p.H), dim3(REC_THREADS), 0, s, p);
    return hipGetLastError();
}
template <bool RG, bool RB, bool NM>
hipError_t disp3(const RecParams& p, bool pt, hipStream_t s) {
    if (pt) return launch_rec<RG, RB, NM, REC_PER_TOKEN_MODE>(p, s);
    return p.S == 1 ? launch_rec<RG, RB, NM, REC_SINGLE>(p, s) : launch_rec<RG, RB, NM, REC_MULTI>(p, s);
}
template <bool RG, bool RB>
hipError_t disp2(const RecParams& p, bool nm, bool pt, hipStream_t s) {
    return nm ? disp3<RG, RB, true>(p, pt, s) : disp3<RG, RB, false>(p, pt, s);
}
template <bool RG>
hipError_t disp1(const RecParams& p, bool rb, bool nm, bool pt, hipStream_t s) {
    return rb ? disp2<RG, true>(p, nm, pt, s) : disp2<RG, false>(p, nm, pt, s);
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace
}  // namespace kda355

using namespace kda355;

extern "C" int kda355_recurrent_launch(const KdaRecurrentArgs* a, kda355_stream_t stream) {
    KDA_CHECK_ARG(a != nullptr, "recurrent: null args");
    const uint32_t f = a->flags;
    const bool per_token = f & KDA355_REC_PER_TOKEN;
    KDA_CHECK_ARG(a->B >= 0 && a->S >= 1 && a->H >= 1, "recurrent: B=%d S=%d H=%d", a->B, a->S, a->H);
    if (a->B == 0) return 0;
    KDA_CHECK_ARG(a->q && a->k && a->v && a->g && a->beta && a->read_pool && a->read_idx && a->out,
                  "recurrent: a required pointer is null");
    KDA_CHECK_ARG(!(f & KDA355_REC_RAW_GATE) || (a->A_log && a->dt_bias), "recurrent: raw gate needs A_log and dt_bias");
    KDA_CHECK_ARG(!per_token || (a->write_pool && a->write_idx), "recurrent: PER_TOKEN needs write_pool and write_idx");
    KDA_CHECK_ARG(a->read_idx_stride >= 1, "recurrent: read_idx_stride must be >= 1");
    KDA_CHECK_ARG(!a->num_accepted || a->read_idx_stride >= a->S, "recurrent: num_accepted needs read_idx_stride >= S");
    // 16-byte state rows, 8-byte bf16 q/k/raw_g quads and 16-byte fp32 g quads are loaded as vectors
    KDA_CHECK_ARG(aligned(a->read_pool, 16) && a->read_slot_stride % 4 == 0, "recurrent: read pool must be 16-byte aligned");
    KDA_CHECK_ARG(!per_token || (aligned(a->write_pool, 16) && a->write_slot_stride % 4 == 0),
                  "recurrent: write pool must be 16-byte aligned");
    KDA_CHECK_ARG(aligned(a->q, 8) && aligned(a->k, 8) && a->qkv_row_stride % 4 == 0, "recurrent: q/k rows must be 8-byte aligned");
    KDA_CHECK_ARG((f & KDA355_REC_RAW_GATE) ? (aligned(a->g, 8) && a->g_row_stride % 4 == 0)
                                             : (aligned(a->g, 16) && a->g_row_stride % 4 == 0),
                  "recurrent: g rows misaligned");
    KDA_CHECK_ARG(aligned(a->out, 4) && a->out_row_stride % 2 == 0, "recurrent: out rows must be 4-byte aligned");
    KDA_CHECK_ARG((int64_t)a->B * a->H < (1ll << 31), "recurrent: grid too large");

    RecParams p;
    p.q = static_cast<const uint16_t*>(a->q);
    p.k = static_cast<const uint16_t*>(a->k);
    p.v = static_cast<const uint16_t*>(a->v);
    p.g = a->g;
    p.beta = a->beta;
    p.A_log = a->A_log;
    p.dt_bias = a->dt_bias;
    p.read_pool = a->read_pool;
    p.write_pool = a->write_pool;
    p.read_idx = a->read_idx;
    p.num_accepted = a->num_accepted;
    p.write_idx = a->write_idx;
    p.out = static_cast<uint16_t*>(a->out);
    p.qkv_rs = a->qkv_row_stride;
    p.g_rs = a->g_row_stride;
    p.beta_rs = a->beta_row_stride;
    p.out_rs = a->out_row_stride;
    p.read_ss = a->read_slot_stride;
    p.read_slots = a->read_slots;
    p.write_ss = a->write_slot_stride;
    p.write_slots = a->write_slots;
    p.B = a->B;
    p.S = a->S;
    p.H = a->H;
    p.read_idx_stride = a->read_idx_stride;
    p.read_min = (f & KDA355_REC_SLOT0_RESERVED) ? 1 : 0;
    p.write_min = (f & KDA355_REC_WRITE_SLOT0_RESERVED) ? 1 : 0;
    p.scale = a->scale;
    p.lb = a->lower_bound;
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool rg = f & KDA355_REC_RAW_GATE, rb = f & KDA355_REC_RAW_BETA, nm = f & KDA355_REC_NORMALIZE_QK;
    const hipError_t e = rg ? disp1<true>(p, rb, nm, per_token, s) : disp1<false>(p, rb, nm, per_token, s);
    if (e != hipSuccess) {
        set_error("recurrent: launch failed: %s", hipGetErrorString(e));
        return KDA355_ELAUNCH;
    }
    return 0;
}

extern "C" int kda355_spec_commit_launch(const KdaSpecCommitArgs* a, kda355_stream_t stream) {
    KDA_CHECK_ARG(a != nullptr, "spec_commit: null args");
    KDA_CHECK_ARG(a->B >= 0 && a->S >= 1 && a->H >= 1, "spec_commit: B=%d S=%d H=%d", a->B, a->S, a->H);
    if (a->B == 0) return 0;
    KDA_CHECK_ARG(a->scratch && a->pool && a->scratch_idx && a->pool_idx && a->num_accepted, "spec_commit: null pointer");
    KDA_CHECK_ARG(aligned(a->scratch, 16) && aligned(a->pool, 16) && a->scratch_slot_stride % 4 == 0 &&
                      a->pool_slot_stride % 4 == 0,
                  "spec_commit: pools must be 16-byte aligned");
    const bool slot0 = (a->flags & KDA355_REC_SLOT0_RESERVED) != 0;
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if ((long long)a->B * a->H * D * D * 4 > WK_STREAM_BYTES)
        hipLaunchKernelGGL(spec_commit_kernel<true>, dim3(a->B * a->H), dim3(WK_THREADS), 0, s, *a, slot0);
    else
        hipLaunchKernelGGL(spec_commit_kernel<false>, dim3(a->B * a->H), dim3(WK_THREADS), 0, s, *a, slot0);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("spec_commit: launch failed: %s", hipGetErrorString(e));
        return KDA355_ELAUNCH;
    }
    return 0;
}
