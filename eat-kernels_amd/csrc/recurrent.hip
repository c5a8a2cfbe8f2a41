// Recurrent KDA decode / speculative verify on gfx950, and the commit of an accepted draft length.
//
// The step is a bandwidth-bound read-modify-write of the fp32 128 x 128 state of each (sequence, head): 64 KiB read,
// 64 KiB written per stored state.  One workgroup of 256 threads (4 wave64) owns one (sequence, head):
//   * lane l of wave w holds state rows  p*16 + w*4 + l/16  (p = 0..7)  and columns  4*(l%16) + {0..3}, 64 + 4*(l%16) + {0..3}
//     -> 64 fp32 registers, each wave load instruction reads 4 rows x 256 contiguous bytes (16-byte lanes);
//   * a state row lives in one group of 16 lanes, so both row reductions (S k and S q) are 4 DPP steps;
//   * o_t = scale * (S' q + u (k . q)) with S' the decayed state before the rank-1 update -- the two reductions are
//     independent, so they are issued together (algebraically the reference's o = scale * S_new q).
// Semantics: kda/mi350x/reference.py:155-171 (recurrent core), slot rules kda/mi350x/kda/decode/kda_v14_b.cu:1013-1042
// (padding slot 0 and out-of-range rows are never read or written; such a sequence's output rows are zero).
#include "common.h"

namespace kda355 {
namespace {

constexpr int REC_THREADS = 256;

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

template <bool RAW_GATE, bool RAW_BETA, bool NORM, bool PER_TOKEN>
__global__ void __launch_bounds__(REC_THREADS) recurrent_kernel(RecParams p) {
    const int bid = blockIdx.x;
    const int n = bid / p.H;
    const int h = bid - n * p.H;
    const int tid = threadIdx.x;
    const int w = tid >> 6;
    const int lane = tid & 63;
    const int grp = lane >> 4;
    const int j = lane & 15;
    const int S = p.S;

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

    // ---- load the state: 8 rows x 8 columns per thread
    const int c0 = 4 * j;
    const float* src = p.read_pool + rd * p.read_ss + (int64_t)h * D * D;
    f32x4 st[8][2];
#pragma unroll
    for (int pp = 0; pp < 8; ++pp) {
        const int row = pp * 16 + w * 4 + grp;
        st[pp][0] = *reinterpret_cast<const f32x4*>(src + row * D + c0);
        st[pp][1] = *reinterpret_cast<const f32x4*>(src + row * D + 64 + c0);
    }

    for (int t = 0; t < S; ++t) {
        const int64_t tok = (int64_t)n * S + t;
        // k, q: columns c0..c0+3 and 64+c0..64+c0+3 (4 bf16 = 8 bytes each)
        const uint16_t* kq_base = p.k + tok * p.qkv_rs + h * D;
        const uint16_t* qq_base = p.q + tok * p.qkv_rs + h * D;
        const u32x2 kb0 = *reinterpret_cast<const u32x2*>(kq_base + c0);
        const u32x2 kb1 = *reinterpret_cast<const u32x2*>(kq_base + 64 + c0);
        const u32x2 qb0 = *reinterpret_cast<const u32x2*>(qq_base + c0);
        const u32x2 qb1 = *reinterpret_cast<const u32x2*>(qq_base + 64 + c0);
        float kk[8], qq[8], dd[8];
        kk[0] = bf2f(kb0.x & 0xffffu); kk[1] = bf2f(kb0.x >> 16); kk[2] = bf2f(kb0.y & 0xffffu); kk[3] = bf2f(kb0.y >> 16);
        kk[4] = bf2f(kb1.x & 0xffffu); kk[5] = bf2f(kb1.x >> 16); kk[6] = bf2f(kb1.y & 0xffffu); kk[7] = bf2f(kb1.y >> 16);
        qq[0] = bf2f(qb0.x & 0xffffu); qq[1] = bf2f(qb0.x >> 16); qq[2] = bf2f(qb0.y & 0xffffu); qq[3] = bf2f(qb0.y >> 16);
        qq[4] = bf2f(qb1.x & 0xffffu); qq[5] = bf2f(qb1.x >> 16); qq[6] = bf2f(qb1.y & 0xffffu); qq[7] = bf2f(qb1.y >> 16);
        if (RAW_GATE) {
            const uint16_t* gb = reinterpret_cast<const uint16_t*>(p.g) + tok * p.g_rs + h * D;
            const u32x2 g0 = *reinterpret_cast<const u32x2*>(gb + c0);
            const u32x2 g1 = *reinterpret_cast<const u32x2*>(gb + 64 + c0);
            const float rg[8] = {bf2f(g0.x & 0xffffu), bf2f(g0.x >> 16), bf2f(g0.y & 0xffffu), bf2f(g0.y >> 16),
                                 bf2f(g1.x & 0xffffu), bf2f(g1.x >> 16), bf2f(g1.y & 0xffffu), bf2f(g1.y >> 16)};
            const float A = __expf(p.A_log[h]);
            const f32x4 db0 = *reinterpret_cast<const f32x4*>(p.dt_bias + h * D + c0);
            const f32x4 db1 = *reinterpret_cast<const f32x4*>(p.dt_bias + h * D + 64 + c0);
            const float db[8] = {db0.x, db0.y, db0.z, db0.w, db1.x, db1.y, db1.z, db1.w};
#pragma unroll
            for (int c = 0; c < 8; ++c) dd[c] = __expf(p.lb * sigmoidf_(A * (rg[c] + db[c])));
        } else {
            const float* gb = reinterpret_cast<const float*>(p.g) + tok * p.g_rs + h * D;
            const f32x4 g0 = *reinterpret_cast<const f32x4*>(gb + c0);
            const f32x4 g1 = *reinterpret_cast<const f32x4*>(gb + 64 + c0);
            dd[0] = __expf(g0.x); dd[1] = __expf(g0.y); dd[2] = __expf(g0.z); dd[3] = __expf(g0.w);
            dd[4] = __expf(g1.x); dd[5] = __expf(g1.y); dd[6] = __expf(g1.z); dd[7] = __expf(g1.w);
        }
        float bt;
        if (RAW_BETA) {
            const uint16_t* bb = reinterpret_cast<const uint16_t*>(p.beta);
            bt = sigmoidf_(bf2f(bb[tok * p.beta_rs + h]));
        } else {
            bt = reinterpret_cast<const float*>(p.beta)[tok * p.beta_rs + h];
        }
        if (NORM) {  // x * rsqrt(sum x^2 + 1e-6)  (kda/mi350x/reference.py:159-160)
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

        // v for this thread's 8 rows
        const uint16_t* vb = p.v + tok * p.qkv_rs + h * D;
        float vv[8];
#pragma unroll
        for (int pp = 0; pp < 8; ++pp) vv[pp] = bf2f(vb[pp * 16 + w * 4 + grp]);

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
        // output: lane j < 8 of each group writes row (j*16 + w*4 + grp)
        {
            float o = ov[0];
#pragma unroll
            for (int pp = 1; pp < 8; ++pp) o = (j == pp) ? ov[pp] : o;
            if (j < 8) p.out[tok * p.out_rs + h * D + j * 16 + w * 4 + grp] = (uint16_t)f2bf(o);
        }
        if (PER_TOKEN) {
            const int64_t wr = p.write_idx[(int64_t)n * S + t];
            if (row_ok(wr, p.write_min, p.write_slots)) {
                float* dst = p.write_pool + wr * p.write_ss + (int64_t)h * D * D;
#pragma unroll
                for (int pp = 0; pp < 8; ++pp) {
                    const int row = pp * 16 + w * 4 + grp;
                    *reinterpret_cast<f32x4*>(dst + row * D + c0) = st[pp][0];
                    *reinterpret_cast<f32x4*>(dst + row * D + 64 + c0) = st[pp][1];
                }
            }
        }
    }
    if (!PER_TOKEN) {
        float* dst = p.read_pool + rd * p.read_ss + (int64_t)h * D * D;
#pragma unroll
        for (int pp = 0; pp < 8; ++pp) {
            const int row = pp * 16 + w * 4 + grp;
            *reinterpret_cast<f32x4*>(dst + row * D + c0) = st[pp][0];
            *reinterpret_cast<f32x4*>(dst + row * D + 64 + c0) = st[pp][1];
        }
    }
}

// Copy one (sequence, head) state: scratch[scratch_idx[n, a-1]] -> pool[pool_idx[n]].
__global__ void __launch_bounds__(256) spec_commit_kernel(KdaSpecCommitArgs a, bool slot0) {
    const int n = blockIdx.x / a.H;
    const int h = blockIdx.x - n * a.H;
    int acc = a.num_accepted[n];
    acc = acc < 1 ? 1 : (acc > a.S ? a.S : acc);
    const int64_t sr = a.scratch_idx[(int64_t)n * a.S + acc - 1];
    const int64_t pr = a.pool_idx[n];
    if (sr < 0 || sr >= a.scratch_slots || pr < (slot0 ? 1 : 0) || pr >= a.pool_slots) return;
    const f32x4* s = reinterpret_cast<const f32x4*>(a.scratch + sr * a.scratch_slot_stride + (int64_t)h * D * D);
    f32x4* d = reinterpret_cast<f32x4*>(a.pool + pr * a.pool_slot_stride + (int64_t)h * D * D);
    f32x4 buf[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) buf[i] = s[i * 256 + threadIdx.x];
#pragma unroll
    for (int i = 0; i < 16; ++i) d[i * 256 + threadIdx.x] = buf[i];
}

template <bool RG, bool RB, bool NM, bool PT>
hipError_t launch_rec(const RecParams& p, hipStream_t s) {
    hipLaunchKernelGGL((recurrent_kernel<RG, RB, NM, PT>), dim3(p.B * p.H), dim3(REC_THREADS), 0, s, p);
    return hipGetLastError();
}
template <bool RG, bool RB, bool NM>
hipError_t disp3(const RecParams& p, bool pt, hipStream_t s) {
    return pt ? launch_rec<RG, RB, NM, true>(p, s) : launch_rec<RG, RB, NM, false>(p, s);
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
    hipLaunchKernelGGL(spec_commit_kernel, dim3(a->B * a->H), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), *a,
                       (a->flags & KDA355_REC_SLOT0_RESERVED) != 0);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("spec_commit: launch failed: %s", hipGetErrorString(e));
        return KDA355_ELAUNCH;
    }
    return 0;
}
