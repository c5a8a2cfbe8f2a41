// The chunk walk on 32-token chunks with a 4-wave workgroup (included by prefill.hip, inside its namespace).
//
// chunk_kernel keeps a 64-token chunk's operands in 156 KiB of LDS, so a CU holds one workgroup: its 8 waves (two
// per SIMD) meet at the same five barriers per chunk and stall together.  Here a chunk is 32 tokens, the row arrays
// halve and the workgroup needs 72 KiB, so two independent workgroups share a CU: still two waves per SIMD, but from
// workgroups whose barriers and dependent chains do not line up.  Per token the work is the same (the Gram and solve
// blocks shrink with the chunk; the per-chunk state work -- decay, fp16 copies of S -- doubles).  Each wave keeps a
// 128 x 32 slice of S (64 VGPRs), so a piece that also carries its transition does not fit: this kernel runs unsplit
// layouts only: the plan picks it (KdaPrefillPlan.chunk32) for layouts whose items outnumber the CUs when its schedule
// model has it finish first, and launches in the precise mode keep chunk_kernel.
//
// Same algorithm, phases and operand conventions as chunk_kernel, with two row blocks of 16 instead of four:
//   P0 raw rows (gate, beta, q / k sums of squares), P1 gate cumsum in 2 segments, P2 element and block factors
//   (7 factor rows), P4 Gram tiles (wave I = 0 / 1: diagonal block I's A_kk with the bf16 hi / lo split, then T_II;
//   wave 2 + I: its A_qk, then one product of block (1, 0)), P5 Q~ and Kd^T layouts (tokens permuted by pos32),
//   P6 W / U (wave w: channel / value tiles 2 w, 2 w + 1),
//   P7 the walk (wave w: S[:, 32 w .. 32 w + 31], K step outermost).  Checkpoints fall on 64-token boundaries, i.e.
//   after every second chunk (or after the last chunk of the sequence).
constexpr int C32_THREADS = 256;
constexpr int RS16T = 40;                                // fp16 rows of 32 (+ 8)
constexpr int C32_A = 0;                                 // gate / Gamma, then k^ fi: fp32 [32][RS32]
constexpr int C32_B = C32_A + 32 * RS32 * 4;             // q^ fi fp32 [32][RS32]; then Q~ fp16 [32][RS16]
constexpr int C32_BV = C32_B + 32 * RS16 * 2;            // W fp16 [32][RS16] (region B's upper half)
constexpr int C32_C = C32_B + 2 * 32 * RS16 * 2;         // k^ fj fp32 [32][RS32]; then Kd^T fp16 [128][RS16T]
constexpr int C32_V = C32_C + 32 * RS32 * 4;             // raw v rows bf16 [32][RS16]
constexpr int C32_AQ = C32_V + 32 * RS16 * 2;            // A_qk fp16 [32][RS16T] (columns permuted)
constexpr int C32_AK = C32_AQ + 32 * RS16T * 2;          // -A_kk block (1, 0) and T_II diagonal blocks fp16 [32][RS16T]
constexpr int C32_GM = C32_AK + 32 * RS16T * 2;          // the cumsum's block middle rows [2][128] fp32
constexpr int C32_F = C32_GM + 2 * 128 * 4;              // factor rows [7][128] fp32
constexpr int C32_WT = C32_F + 7 * 128 * 4;              // segment totals [2][128] fp32
constexpr int C32_BETA = C32_WT + 2 * 128 * 4;           // [32] fp32
constexpr int C32_DT = C32_BETA + 32 * 4;                // An dt_bias [128] fp32 (gate in the kernel)
constexpr int C32_L = C32_DT + 128 * 4;                  // A_kk diagonal blocks, column-major [2][16][20] fp32
constexpr int C32_TOTAL = C32_L + 2 * 16 * 20 * 4;
static_assert(32 * RS32 * 4 <= 2 * 32 * RS16 * 2, "q^ fi fits region B");
static_assert(128 * RS16T * 2 <= 32 * RS32 * 4, "Kd^T fits region C");
static_assert(2 * C32_TOTAL <= 160 * 1024, "two workgroups per CU");
// factor rows: a_1 = e^{Gamma_m(1) - Gamma_15}, b_10 = e^{Gamma_15 - Gamma_m(0)}, x_I = e^{Gamma_m(I)},
// y_I = e^{Gamma_c - Gamma_m(I)}, e^{Gamma_c} (Gamma_m(I): the middle row 16 I + 7 of block I; Gamma_c: the last row)
constexpr int F32_A = 0, F32_B = 1, F32_X = 2, F32_Y = 4, F32_DEC = 6;

// S slice of this lane (k = 16 dt + 4 g .. + 3, v = 32 w + 16 ct + m) to a V-major [128][128] fp32 / bf16 state
__device__ __forceinline__ void store_state32(float* dst, const f32x4 (&S)[8][2], int w, int g, int m) {
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        float* row = dst + (32 * w + 16 * ct + m) * D + 4 * g;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(row + 16 * dt) = S[dt][ct];
    }
}
__device__ __forceinline__ void store_state32_bf16(uint16_t* dst, const f32x4 (&S)[8][2], int w, int g, int m) {
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        uint16_t* row = dst + (32 * w + 16 * ct + m) * D + 4 * g;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
            *reinterpret_cast<u32x2*>(row + 16 * dt) =
                u32x2{f2bf2(S[dt][ct][0], S[dt][ct][1]), f2bf2(S[dt][ct][2], S[dt][ct][3])};
    }
}

template <bool RG>
__global__ void __launch_bounds__(C32_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
    chunk32_kernel(PfParams p, const int32_t* __restrict__ tab, const int32_t* __restrict__ ck_idx, int list_off) {
    extern __shared__ __align__(16) unsigned char lds[];
    float* sG = reinterpret_cast<float*>(lds + C32_A);
    float* sKA = sG;
    float* sQA = reinterpret_cast<float*>(lds + C32_B);
    half_t* sQt = reinterpret_cast<half_t*>(lds + C32_B);
    half_t* sW = reinterpret_cast<half_t*>(lds + C32_BV);
    float* sKB = reinterpret_cast<float*>(lds + C32_C);
    half_t* sKd = reinterpret_cast<half_t*>(lds + C32_C);
    const uint16_t* sV = reinterpret_cast<const uint16_t*>(lds + C32_V);
    half_t* sAq = reinterpret_cast<half_t*>(lds + C32_AQ);
    half_t* sAk = reinterpret_cast<half_t*>(lds + C32_AK);
    float* sL = reinterpret_cast<float*>(lds + C32_L);
    float* sF = reinterpret_cast<float*>(lds + C32_F);
    float* sWt = reinterpret_cast<float*>(lds + C32_WT);
    float* sGM = reinterpret_cast<float*>(lds + C32_GM);
    float* sBeta = reinterpret_cast<float*>(lds + C32_BETA);
    float* sDT = reinterpret_cast<float*>(lds + C32_DT);

    const int H = p.H;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const bool pool = (p.flags & KDA355_PF_POOL) != 0;
    const bool RB = (p.flags & KDA355_PF_RAW_BETA) != 0;
    const bool NORM = (p.flags & KDA355_PF_NORMALIZE_QK) != 0;
    const int ck_mode = (p.flags & KDA355_PF_CK_EVERY) ? 2 : ((p.flags & KDA355_PF_CK_SINGLE) ? 1 : 0);
    const int every = tab[H_EVERY];
    // one (chain entry, head) item per workgroup; an unsplit layout's entries are whole sequences
    const int item = (int)blockIdx.x;
    const int ci = item / H;
    const int h = item - ci * H;
    const int32_t* en = tab + list_off + C_WORDS * ci;
    const int n = en[C_SEQ], tstart = en[C_TSTART], len = en[C_LEN], pflags = en[C_FLAGS];
    const int first = en[C_FIRST], seqch = en[C_SEQCH], ck_row0 = en[C_CKROW0];
    const int ck_single = (ck_mode == 1) ? en[C_CKSINGLE] : 0;
    const int nch = (len + 31) >> 5;
    int64_t prow = -1;
    const float* src = nullptr;
    if (pool) {
        prow = p.state_idx[n];
        src = (prow >= 0 && prow < p.state_slots && p.has_init[n] != 0)
                  ? p.state_pool + prow * p.state_ss + (int64_t)h * D * D : nullptr;
    } else {
        src = p.init_state ? p.init_state + ((int64_t)n * H + h) * D * D : nullptr;
    }
    int tid = threadIdx.x, lane = tid & 63, m = lane & 15, g = lane >> 4, r = tid >> 3, cb = tid & 7;
    const float dtb = RG ? p.dt_bias[h * D + (tid & (D - 1))] : 0.f;
    const float alog = RG ? p.A_log[h] : 0.f;
    RawRow nx;
    load_row<RG>(p, h, tstart, nch > 0 ? min(32, len) : 0, r, cb, RB, nx);  // an empty sequence loads nothing
    f32x4 S[8][2];
    {
        // through a descriptor of no records when there is no start state; base and size wave-uniform
        const int nrec = __builtin_amdgcn_readfirstlane(src ? D * D * 4 : 0);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            uniform_ptr(src ? static_cast<const void*>(src) : static_cast<const void*>(p.q)), (short)0, nrec, 0x00020000);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int voff = ((32 * w + 16 * ct + m) * D + 4 * g) * 4;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt)
                S[dt][ct] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 64 * dt, 0, 0));
        }
    }
    auto ck_store = [&](int64_t rr) {
        if (rr < 0 || rr >= p.ck_slots) return;
        if (p.ck_bf16)
            store_state32_bf16(reinterpret_cast<uint16_t*>(p.ck_pool) + rr * p.ck_ss + (int64_t)h * D * D, S, w, g, m);
        else
            store_state32(reinterpret_cast<float*>(p.ck_pool) + rr * p.ck_ss + (int64_t)h * D * D, S, w, g, m);
    };
    float An = 0.f;
    if (RG) {
        An = gate_an(alog);
        if (tid < D) sDT[tid] = An * dtb;
    }
    // A_qk block (0, 1) is read by the walk and never written by the Gram phase
    sAq[(tid >> 4) * RS16T + pos32(16 + (tid & 15))] = (half_t)0.f;
    lds_barrier();

    for (int cl = 0; cl < nch; ++cl) {
        // lane indices re-derived every chunk from an opaque copy (recomputed where used, not kept live)
        tid = threadIdx.x;
        asm volatile("" : "+v"(tid));
        lane = tid & 63;
        m = lane & 15;
        g = lane >> 4;
        r = tid >> 3;
        cb = tid & 7;
        const int t0 = tstart + 32 * cl, L = min(32, len - 32 * cl);
        const bool pf = cl + 1 < nch;
        const int pf_t = t0 + 32, pf_L = pf ? min(32, len - 32 * (cl + 1)) : 0;
        // ================= P0: raw rows (v to LDS; gate, beta; q / k sums of squares)
        *reinterpret_cast<u32x4*>(lds + C32_V + r * (2 * RS16) + 32 * cb) = nx.v[0];
        *reinterpret_cast<u32x4*>(lds + C32_V + r * (2 * RS16) + 32 * cb + 16) = nx.v[1];
        float gv[16];
        if (RG) {
            float rg[16];
            const u32x4 gg[2] = {nx.g[0], nx.g[1]};
            unpack16(gg, rg);
            const float lbm = (r < L) ? p.lb * LOG2E : 0.f;
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const f32x4 adt4 = *reinterpret_cast<const f32x4*>(&sDT[16 * cb + 4 * q4]);
#pragma unroll
                for (int ee = 0; ee < 4; ++ee)
                    gv[4 * q4 + ee] =
                        clamp_decay2(lbm * __builtin_amdgcn_rcpf(1.0f + exp2_(fmaf(An, rg[4 * q4 + ee], adt4[ee]))));
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) gv[4 * i + j] = clamp_decay(__uint_as_float(nx.g[i][j]));
        }
        const float bx = RB ? sigmoid_rcp(bf2f(nx.beta)) : __uint_as_float(nx.beta);
        const float bt = (r >= L) ? 0.f : bx;
        float rq = 1.f, rk = 1.f;
        if (NORM) {  // F.normalize(x, eps=1e-6)  (kda/mi350x/reference.py:59-60)
            float sq = 0.f, sk = 0.f;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t wq = nx.q[i][j], wk = nx.k[i][j];  // element copies (see chunk_kernel)
                    const bf16x2_t qp = __builtin_bit_cast(bf16x2_t, wq);
                    const bf16x2_t kp = __builtin_bit_cast(bf16x2_t, wk);
                    sq = __builtin_amdgcn_fdot2_f32_bf16(qp, qp, sq, false);
                    sk = __builtin_amdgcn_fdot2_f32_bf16(kp, kp, sk, false);
                }
            sq = sum8(sq);
            sk = sum8(sk);
            rq = __builtin_amdgcn_rsqf(fmaxf(sq, 1e-12f));
            rk = __builtin_amdgcn_rsqf(fmaxf(sk, 1e-12f));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<f32x4*>(&sG[r * RS32 + 16 * cb + 4 * (i ^ (cb >> 1))]) =
                f32x4{gv[4 * i], gv[4 * i + 1], gv[4 * i + 2], gv[4 * i + 3]};
        if (cb == 0) sBeta[r] = bt;
        lds_barrier();
        // ================= P1: gate cumsum inside the 2 segments of 16 rows
        {
            const int c = tid & 127, s = tid >> 7;
            float x[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = sG[(16 * s + i) * RS32 + swz(c)];
            if (RG) {
#pragma unroll
                for (int i = 1; i < 16; ++i) x[i] += x[i - 1];
            } else {
                x[0] *= LOG2E;
#pragma unroll
                for (int i = 1; i < 16; ++i) x[i] = fmaf(x[i], LOG2E, x[i - 1]);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) sG[(16 * s + i) * RS32 + swz(c)] = x[i];
            sWt[s * 128 + c] = x[15];
            sGM[s * 128 + c] = x[7];
        }
        lds_barrier();
        // ================= P2: element factors (raw threads) and the 7 block-factor rows (channel threads)
        {
            float qf[16], kf[16];
            {
                const u32x4 a[2] = {nx.q[0], nx.q[1]}, b[2] = {nx.k[0], nx.k[1]};
                unpack16(a, qf);
                unpack16(b, kf);
            }
            if (NORM) {
#pragma unroll
                for (int c = 0; c < 16; ++c) { kf[c] *= rk; qf[c] *= rq; }
            }
            const int I = r >> 4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int o = r * RS32 + 16 * cb + 4 * (i ^ (cb >> 1));
                const f32x4 a = *reinterpret_cast<const f32x4*>(&sG[o]);
                const f32x4 b = *reinterpret_cast<const f32x4*>(&sGM[I * 128 + 16 * cb + 4 * i]);
                f32x4 kfi, kfj, qfi;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int c = 4 * i + j;
                    const float d = a[j] - b[j];
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
            const int c = tid & 127, qd = __builtin_amdgcn_readfirstlane(tid >> 7);  // wave-uniform
            const float o1 = sWt[c];
            // Gamma at rows 7, 15, 23, 31
            const float gr0 = sGM[c], gr1 = o1, gr2 = sGM[128 + c] + o1, gr3 = sWt[128 + c] + o1;
            if (qd == 0) {
                sF[F32_A * 128 + c] = exp2_(gr2 - gr1);
                sF[F32_X * 128 + c] = exp2_(gr0);
                sF[(F32_Y + 1) * 128 + c] = exp2_(gr3 - gr2);
                sF[F32_DEC * 128 + c] = exp2_(gr3);
            } else {
                sF[F32_B * 128 + c] = exp2_(gr1 - gr0);
                sF[(F32_X + 1) * 128 + c] = exp2_(gr2);
                sF[F32_Y * 128 + c] = exp2_(gr3 - gr0);
            }
        }
        lds_barrier();
        // ================= P4: Gram tiles.  Wave I (0, 1): the diagonal block's A_kk (bf16 hi + lo products of
        // k^ fi and k^ fj), then T_II = (I + L_II)^-1; wave 2 + I: the same block's A_qk (k^ fj and q^ fi), then one
        // product of block (1, 0) from fp16 operands <= 1 (reference row 15): A_kk on wave 2, A_qk on wave 3.
        {
            const int I = w & 1, i = 16 * I + m;
            const bool kk = w < 2;  // wave-uniform
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            const float* sX = kk ? sKA : sQA;  // the product's second operand: k^ fi (A_kk) or q^ fi (A_qk)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int c0 = 32 * s + 8 * g;
                uint32_t xh[4], xl[4], kbh[4], kbl[4];
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    const f32x4 xa = *reinterpret_cast<const f32x4*>(&sX[i * RS32 + swz(c0 + 4 * hf)]);
                    const f32x4 kb = *reinterpret_cast<const f32x4*>(&sKB[i * RS32 + swz(c0 + 4 * hf)]);
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int ee = 2 * hf + j;
                        split_bf16x2(xa[2 * j], xa[2 * j + 1], xh[ee], xl[ee]);
                        split_bf16x2(kb[2 * j], kb[2 * j + 1], kbh[ee], kbl[ee]);
                    }
                }
                const bf16x8 Xh = as_bf16x8(xh), Xl = as_bf16x8(xl), Kbh = as_bf16x8(kbh), Kbl = as_bf16x8(kbl);
                if (kk) {  // A_kk: lane (g, m) holds row 16 I + 4 g + e, column 16 I + m
                    acc = mfma32bf(Xh, Kbh, acc);
                    acc = mfma32bf(Xh, Kbl, acc);
                    acc = mfma32bf(Xl, Kbh, acc);
                } else {   // A_qk transposed: lane (g, m) holds row 16 I + m, columns 16 I + 4 g .. + 3
                    acc = mfma32bf(Kbh, Xh, acc);
                    acc = mfma32bf(Kbl, Xh, acc);
                    acc = mfma32bf(Kbh, Xl, acc);
                }
            }
            if (kk) {
                f32x4 lt;
                const f32x4 bt4 = *reinterpret_cast<const f32x4*>(&sBeta[16 * I + 4 * g]);
#pragma unroll
                for (int ee = 0; ee < 4; ++ee) lt[ee] = (m < 4 * g + ee) ? bt4[ee] * acc[ee] : 0.f;
                *reinterpret_cast<f32x4*>(&sL[(I * 16 + m) * 20 + 4 * g]) = lt;
                const float* Lb = sL + I * 16 * 20;  // column k of L_II is the contiguous row k; the wave reads back
                float x[16];                         // what it has just written (its LDS operations complete in order)
#pragma unroll
                for (int ii = 0; ii < 16; ++ii) x[ii] = (ii == m) ? 1.f : 0.f;
#pragma unroll
                for (int k = 0; k < 15; ++k) {
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
                    for (int ii = 0; ii < 16; ++ii) sAk[(16 * I + ii) * RS16T + 16 * I + m] = (half_t)x[ii];
                }
            } else {
                f16x4 aq;
#pragma unroll
                for (int ee = 0; ee < 4; ++ee) aq[ee] = (half_t)((4 * g + ee <= m) ? acc[ee] : 0.f);  // causal
                *reinterpret_cast<f16x4*>(&sAq[i * RS16T + pos32(16 * I + 4 * g)]) = aq;
            }
        }
        if (w >= 2) {  // block (1, 0): wave 2 A_kk, wave 3 A_qk (transposed tiles: lane (g, m) holds row 16 + m,
                       // columns 4 g .. + 3)
            const bool kk = w == 2;
            const int i = 16 + m;
            const float* sX = kk ? sKA : sQA;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int c0 = 32 * s + 8 * g;
                f16x8 xa, kb;
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    const f32x4 a = *reinterpret_cast<const f32x4*>(&sX[i * RS32 + swz(c0 + 4 * hf)]);
                    const f32x4 fa = *reinterpret_cast<const f32x4*>(&sF[F32_A * 128 + c0 + 4 * hf]);
                    const f32x4 b = *reinterpret_cast<const f32x4*>(&sKB[m * RS32 + swz(c0 + 4 * hf)]);
                    const f32x4 fb = *reinterpret_cast<const f32x4*>(&sF[F32_B * 128 + c0 + 4 * hf]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        xa[4 * hf + j] = (half_t)(a[j] * fa[j]);
                        kb[4 * hf + j] = (half_t)(b[j] * fb[j]);
                    }
                }
                acc = mfma32(kb, xa, acc);
            }
            if (kk) {
                const float nb = -sBeta[i];
                f16x4 ak;
#pragma unroll
                for (int ee = 0; ee < 4; ++ee) ak[ee] = (half_t)(nb * acc[ee]);
                *reinterpret_cast<f16x4*>(&sAk[i * RS16T + 4 * g]) = ak;
            } else {
                f16x4 aq;
#pragma unroll
                for (int ee = 0; ee < 4; ++ee) aq[ee] = (half_t)acc[ee];
                *reinterpret_cast<f16x4*>(&sAq[i * RS16T + pos32(4 * g)]) = aq;
            }
        }
        // ================= P5: Q~, Kd^T into their walk layouts (raw threads)
        // the start state's loads complete here in the first chunk (an empty use of S), not before a later walk
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) asm volatile("" : "+v"(S[dt][ct]));
        if (pf) load_row_qk(p, h, pf_t, pf_L, r, cb, nx);
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
                const f32x4 xf = *reinterpret_cast<const f32x4*>(&sF[(F32_X + I) * 128 + 16 * cb + 4 * gq]);
                f16x4 o;
#pragma unroll
                for (int ee = 0; ee < 4; ++ee) o[ee] = (half_t)(qfi[4 * gq + ee] * xf[ee]);
                *reinterpret_cast<f16x4*>(&sQt[r * RS16 + 32 * blk + 8 * gq + 4 * hb]) = o;
            }
            const int pr = pos32(r);
#pragma unroll
            for (int ee = 0; ee < 16; ++ee) {
                const float y = sF[(F32_Y + I) * 128 + 16 * cb + ee];
                sKd[(16 * cb + (ee ^ cb)) * RS16T + pr] = (half_t)(kfj[ee] * y);
            }
        }
        // ================= P6: W and U by block forward substitution (wave w: channel / value tiles 2 w, 2 w + 1)
        if (pf) load_row_vb(p, h, pf_t, pf_L, r, cb, RB, nx);
        f32x4 Ur[2][2];  // [block I][tile t]: U[token 16 I + 4 g + e][value 32 w + 16 t + m]
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int c = 16 * (2 * w + t) + m;
            f32x4 Xw[2];
            f16x4 Xh0, Uh0;
#pragma unroll
            for (int I = 0; I < 2; ++I) {
                const float xI = sF[(F32_X + I) * 128 + c];
                const f32x4 b4 = *reinterpret_cast<const f32x4*>(&sBeta[16 * I + 4 * g]);
                f32x4 aw, au;
#pragma unroll
                for (int ee = 0; ee < 4; ++ee) {
                    const int rw = 16 * I + 4 * g + ee;
                    aw[ee] = b4[ee] * sKA[rw * RS32 + swz(c)] * xI;
                    au[ee] = b4[ee] * bf2f(sV[rw * RS16 + c]);
                }
                if (I == 1) {
                    const f16x4 A = *reinterpret_cast<const f16x4*>(&sAk[(16 + m) * RS16T + 4 * g]);
                    aw = mfma16(A, Xh0, aw);
                    au = mfma16(A, Uh0, au);
                }
                const f16x4 T = *reinterpret_cast<const f16x4*>(&sAk[(16 * I + m) * RS16T + 16 * I + 4 * g]);
                f16x4 bwh, buh;
#pragma unroll
                for (int ee = 0; ee < 4; ++ee) { bwh[ee] = (half_t)aw[ee]; buh[ee] = (half_t)au[ee]; }
                const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                Xw[I] = mfma16(T, bwh, z);
                Ur[I][t] = mfma16(T, buh, z);
                if (I == 0) {
#pragma unroll
                    for (int ee = 0; ee < 4; ++ee) { Xh0[ee] = (half_t)Xw[0][ee]; Uh0[ee] = (half_t)Ur[0][t][ee]; }
                }
            }
            const int pc = 32 * (c >> 5) + pos32(c & 31);
#pragma unroll
            for (int I = 0; I < 2; ++I)
#pragma unroll
                for (int ee = 0; ee < 4; ++ee) sW[(16 * I + 4 * g + ee) * RS16 + pc] = (half_t)Xw[I][ee];
        }
        lds_barrier();
        // ================= P7: the walk (wave w: S[:, 32 w .. 32 w + 31])
        if (pf) load_row_g<RG>(p, h, pf_t, pf_L, r, cb, nx);
        // every-n row 0: the state before the sequence's first token
        if (cl == 0 && ck_mode == 2 && every > 0 && first == 0) ck_store(ck_idx[ck_row0]);
        {
            f16x8 SB[4][2];
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                    for (int ee = 0; ee < 4; ++ee) {
                        SB[s][ct][ee] = (half_t)S[2 * s][ct][ee];
                        SB[s][ct][4 + ee] = (half_t)S[2 * s + 1][ct][ee];
                    }
            f32x4 Vp[2][2];  // W S, K step outermost
#pragma unroll
            for (int it = 0; it < 2; ++it)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) Vp[it][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int it = 0; it < 2; ++it) {
                    const f16x8 A = *reinterpret_cast<const f16x8*>(&sW[(16 * it + m) * RS16 + 32 * s + 8 * g]);
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct) Vp[it][ct] = mfma32(A, SB[s][ct], Vp[it][ct]);
                }
            f16x8 VB[2];  // V' = U - W S as fp16, tokens 4 g + e and 16 + 4 g + e
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int ee = 0; ee < 4; ++ee) {
                    VB[ct][ee] = (half_t)(Ur[0][ct][ee] - Vp[0][ct][ee]);
                    VB[ct][4 + ee] = (half_t)(Ur[1][ct][ee] - Vp[1][ct][ee]);
                }
            // O^T = S^T Q~^T + V'^T A_qk^T (lane (g, m): token 16 it + m, values 32 w + 16 ct + 4 g .. + 3)
            f32x4 ao[2][2];
#pragma unroll
            for (int it = 0; it < 2; ++it)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) ao[it][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int it = 0; it < 2; ++it) {
                    const f16x8 B = *reinterpret_cast<const f16x8*>(&sQt[(16 * it + m) * RS16 + 32 * s + 8 * g]);
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct) ao[it][ct] = mfma32(SB[s][ct], B, ao[it][ct]);
                }
#pragma unroll
            for (int it = 0; it < 2; ++it) {
                const f16x8 B = *reinterpret_cast<const f16x8*>(&sAq[(16 * it + m) * RS16T + 8 * g]);
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) ao[it][ct] = mfma32(VB[ct], B, ao[it][ct]);
            }
#pragma unroll
            for (int it = 0; it < 2; ++it)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
                    const u32x2 o = {f2bf2(p.scale * ao[it][ct][0], p.scale * ao[it][ct][1]),
                                     f2bf2(p.scale * ao[it][ct][2], p.scale * ao[it][ct][3])};
                    if (16 * it + m < L)
                        *reinterpret_cast<u32x2*>(p.out + ((int64_t)t0 + 16 * it + m) * p.out_rs + (int64_t)h * D +
                                                  32 * w + 16 * ct + 4 * g) = o;
                }
            // S <- diag(e^{Gamma_c}) S + Kd^T V'
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
                const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sF[F32_DEC * 128 + 16 * dt + 4 * g]);
                const f16x8 A = *reinterpret_cast<const f16x8*>(&sKd[(16 * dt + (m ^ dt)) * RS16T + 8 * g]);
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
#pragma unroll
                    for (int ee = 0; ee < 4; ++ee) S[dt][ct][ee] *= d4[ee];
                    S[dt][ct] = mfma32(A, VB[ct], S[dt][ct]);
                }
            }
        }
        // checkpoints at 64-token boundaries: after every second chunk, and after the sequence's last chunk
        if ((cl & 1) || cl + 1 == nch) {
            const int cs = first + ((cl + 2) >> 1);
            if (ck_mode == 1 && cs == ck_single) ck_store(ck_idx[n]);
            if (ck_mode == 2 && every > 0 && cs % every == 0 && cs < seqch) ck_store(ck_idx[ck_row0 + cs / every]);
        }
        // no barrier here: the walk writes no LDS and reads nothing the next raw-row phase writes
    }
    if (pflags & PIECE_LAST) {
        if (pool) {
            if (prow >= 0 && prow < p.state_slots) store_state32(p.state_pool + prow * p.state_ss + (int64_t)h * D * D, S, w, g, m);
        } else {
            store_state32(p.final_state + ((int64_t)n * H + h) * D * D, S, w, g, m);
        }
    }
}

template <bool RG>
hipError_t launch_chunk32(const PfParams& p, int list_off, int wgs, hipStream_t s) {
    static bool attr_set = false;  // idempotent; a race only repeats the call
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(chunk32_kernel<RG>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, C32_TOTAL);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL((chunk32_kernel<RG>), dim3(wgs), dim3(C32_THREADS), C32_TOTAL, s, p, p.tab, p.ck_idx, list_off);
    return hipGetLastError();
}
