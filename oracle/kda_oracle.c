/*
 * kda_oracle.c -- CPU restatement of the KDA reference recurrences.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP kernels are compared against, and the CPU
 * baseline that bench.py times next to them.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product library (libkda355.so) never links or calls it.
 *
 * What it restates (reference paths relative to caoshiyi/eat-kernels):
 *   kdao_gate            kda/mi350x/reference.py:19-22        g = lb * sigmoid(exp(A_log[h]) * (raw_g + dt_bias[h,k]))
 *   kdao_l2norm_clamp    kda/mi350x/reference.py:59-60        F.normalize(x, eps=1e-6) = x / max(|x|, eps)
 *   kdao_l2norm_rsqrt    kda/mi350x/reference.py:159-160      x * rsqrt(sum x^2 + eps) * mult   (decode form)
 *   kdao_sigmoid         kda/mi350x/reference.py:63,163       beta = sigmoid(raw_beta)
 *   kdao_prefill         kda/mi350x/reference.py:79-100       token recurrence per (sequence, head):
 *                        kda/mi350x_plain/reference.py:30-38      S <- S * exp(g_t)  (key rows)
 *                        kda/b200/reference.py:30-37              u  = beta_t (v_t - k_t^T S)
 *                                                                 S <- S + k_t u^T
 *                                                                 o_t = scale * q_t^T S
 *                        plus state snapshots "after the first o tokens" of a sequence, which covers both the
 *                        MI350X single checkpoint (reference.py:52-57,90-91) and the B200 every-n rows
 *                        (kda/b200/test_kda_b200.py:38-55: row j = state before token j*n = after j*n tokens).
 *   kdao_recurrent       kda/mi350x/reference.py:155-171      decode / spec-verify core on the V-major state
 *                                                             st[v,k]; state after every token returned.
 *
 * Layouts: the pool / state tensors are V-major [.., 128(V), 128(K)] as in reference.py:9.  Internally the
 * prefill chain keeps S K-major [K][V] exactly as reference.py:79 does.
 * Precision: every function exists in fp32 (the reference's dtype=torch.float32 path) and fp64 (the fp64
 * recurrence of kda/b200/reference.py).  Summation order is the plain left-to-right loop; torch's einsum
 * order is not reproduced bit for bit (results agree to fp32 rounding).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define D 128

/* ------------------------------------------------------------------------------------------ elementwise */

/* reference.py:19-22 (fp32 path: every operand is converted to fp32 first). */
void kdao_gate(const float* raw_g, const float* A_log, const float* dt_bias, float lower_bound, int64_t T, int H,
               float* g_out) {
    for (int64_t t = 0; t < T; ++t)
        for (int h = 0; h < H; ++h) {
            const float a = expf(A_log[h]);
            for (int k = 0; k < D; ++k) {
                const int64_t i = (t * H + h) * D + k;
                const float x = a * (raw_g[i] + dt_bias[h * D + k]);
                g_out[i] = lower_bound * (1.0f / (1.0f + expf(-x)));
            }
        }
}

void kdao_sigmoid(const float* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = 1.0f / (1.0f + expf(-x[i]));
}

/* reference.py:59-60: F.normalize(x, dim=-1, eps) = x / max(||x||_2, eps), rows of 128. */
void kdao_l2norm_clamp(const float* x, int64_t rows, float eps, float* y) {
    for (int64_t r = 0; r < rows; ++r) {
        double ss = 0.0;
        for (int k = 0; k < D; ++k) ss += (double)x[r * D + k] * x[r * D + k];
        float nrm = (float)sqrt(ss);
        if (nrm < eps) nrm = eps;
        for (int k = 0; k < D; ++k) y[r * D + k] = x[r * D + k] / nrm;
    }
}

/* reference.py:159-160: x * rsqrt(sum x^2 + eps) * mult (mult = 128^-0.5 for q, 1 for k). */
void kdao_l2norm_rsqrt(const float* x, int64_t rows, float eps, float mult, float* y) {
    for (int64_t r = 0; r < rows; ++r) {
        float ss = 0.0f;
        for (int k = 0; k < D; ++k) ss += x[r * D + k] * x[r * D + k];
        const float inv = 1.0f / sqrtf(ss + eps);
        for (int k = 0; k < D; ++k) y[r * D + k] = x[r * D + k] * inv * mult;
    }
}

/* ------------------------------------------------------------------------------------------ prefill chain */

/* One (sequence, head) chain over tokens [0, len) in precision REAL.  Pointers are pre-offset to the
 * sequence's first token and the head; q/k/v/g rows are `ts` floats apart, beta entries `bs` apart.
 * S is K-major [K][V] (reference.py:79), updated in place.  snap_at: ascending token counts (ns of them)
 * after which the V-major state is copied to snaps + j*snap_stride. */
#define DEFINE_CHAIN(NAME, REAL, EXP)                                                                          \
    static void NAME(const float* q, const float* k, const float* v, const float* g, const float* beta,       \
                     int64_t ts, int64_t bs, int64_t len, double scale, REAL* S, float* o,                    \
                     const int64_t* snap_at, int ns, float* snaps, int64_t snap_stride) {                      \
        REAL dec[D], kk[D], qq[D], kS[D], u[D], acc[D];                                                        \
        int sj = 0;                                                                                            \
        for (; sj < ns && snap_at[sj] == 0; ++sj)                                                              \
            for (int a = 0; a < D; ++a)                                                                        \
                for (int b = 0; b < D; ++b) snaps[sj * snap_stride + b * D + a] = (float)S[a * D + b];         \
        for (int64_t t = 0; t < len; ++t) {                                                                    \
            const float* qt = q + t * ts; const float* kt = k + t * ts;                                        \
            const float* vt = v + t * ts; const float* gt = g + t * ts;                                        \
            const REAL bt = (REAL)beta[t * bs];                                                                \
            for (int a = 0; a < D; ++a) { dec[a] = EXP((REAL)gt[a]); kk[a] = kt[a]; qq[a] = qt[a]; }           \
            /* S <- S * exp(g): scales key rows (reference.py:86) */                                           \
            for (int a = 0; a < D; ++a) for (int b = 0; b < D; ++b) S[a * D + b] *= dec[a];                   \
            /* kS = k^T S (reference.py:87) */                                                                 \
            for (int b = 0; b < D; ++b) kS[b] = 0;                                                             \
            for (int a = 0; a < D; ++a) for (int b = 0; b < D; ++b) kS[b] += kk[a] * S[a * D + b];            \
            /* S += k (beta (v - kS))^T (reference.py:88) */                                                   \
            for (int b = 0; b < D; ++b) u[b] = bt * ((REAL)vt[b] - kS[b]);                                     \
            for (int a = 0; a < D; ++a) for (int b = 0; b < D; ++b) S[a * D + b] += kk[a] * u[b];             \
            /* o = scale q^T S (reference.py:89) */                                                            \
            for (int b = 0; b < D; ++b) acc[b] = 0;                                                            \
            for (int a = 0; a < D; ++a) for (int b = 0; b < D; ++b) acc[b] += qq[a] * S[a * D + b];           \
            for (int b = 0; b < D; ++b) o[t * ts + b] = (float)((REAL)scale * acc[b]);                         \
            for (; sj < ns && snap_at[sj] == t + 1; ++sj)                                                      \
                for (int a = 0; a < D; ++a)                                                                    \
                    for (int b = 0; b < D; ++b) snaps[sj * snap_stride + b * D + a] = (float)S[a * D + b];     \
        }                                                                                                      \
    }

DEFINE_CHAIN(chain_f32, float, expf)
DEFINE_CHAIN(chain_f64, double, exp)

/*
 * Varlen prefill over N sequences, H heads (reference.py:25-101 with the pool indirection done by the caller).
 *   q, k, v, g : [T, H, 128] fp32 (q, k already normalized; g is the log-decay; beta already activated)
 *   beta       : [T, H]
 *   cu         : [N+1] int64 token offsets
 *   S0         : [N, H, 128, 128] V-major initial states, or NULL (zeros)
 *   S_fin      : [N, H, 128, 128] V-major final states (written)
 *   out        : [T, H, 128] outputs (written)
 *   snap_at    : [N, max_snaps] token counts (ascending, -1 = unused) after which a snapshot is taken, or NULL
 *   snaps      : [N, max_snaps, H, 128, 128] V-major snapshots (written where snap_at >= 0)
 *   precision  : 32 or 64;  nthreads: OpenMP threads (<= 0: runtime default)
 * Returns 0, or -1 for bad arguments.
 */
int kdao_prefill(const float* q, const float* k, const float* v, const float* g, const float* beta, int64_t T, int H,
                 const int64_t* cu, int N, double scale, const float* S0, float* S_fin, float* out,
                 const int64_t* snap_at, int max_snaps, float* snaps, int precision, int nthreads) {
    if (H <= 0 || N < 0 || (precision != 32 && precision != 64)) return -1;
    if (cu[0] != 0 || cu[N] != T) return -1;
    const int64_t pairs = (int64_t)N * H;
    const int64_t ts = (int64_t)H * D;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
#endif
    for (int64_t p = 0; p < pairs; ++p) {
        const int n = (int)(p / H), h = (int)(p % H);
        const int64_t t0 = cu[n], len = cu[n + 1] - cu[n];
        int ns = 0;
        const int64_t* sa = snap_at ? snap_at + (int64_t)n * max_snaps : NULL;
        if (sa) while (ns < max_snaps && sa[ns] >= 0) ++ns;
        float* sn = snaps ? snaps + ((int64_t)n * max_snaps * H + h) * D * D : NULL;
        const int64_t sstride = (int64_t)H * D * D;
        const float* init = S0 ? S0 + ((int64_t)n * H + h) * D * D : NULL;
        float* fin = S_fin + ((int64_t)n * H + h) * D * D;
        const int64_t off = t0 * ts + (int64_t)h * D;
        if (precision == 64) {
            double* S = (double*)malloc(sizeof(double) * D * D);
            for (int a = 0; a < D; ++a)
                for (int b = 0; b < D; ++b) S[a * D + b] = init ? (double)init[b * D + a] : 0.0;
            chain_f64(q + off, k + off, v + off, g + off, beta + t0 * H + h, ts, H, len, scale, S, out + off, sa, ns,
                      sn, sstride);
            for (int a = 0; a < D; ++a)
                for (int b = 0; b < D; ++b) fin[b * D + a] = (float)S[a * D + b];
            free(S);
        } else {
            float* S = (float*)malloc(sizeof(float) * D * D);
            for (int a = 0; a < D; ++a)
                for (int b = 0; b < D; ++b) S[a * D + b] = init ? init[b * D + a] : 0.0f;
            chain_f32(q + off, k + off, v + off, g + off, beta + t0 * H + h, ts, H, len, scale, S, out + off, sa, ns,
                      sn, sstride);
            for (int a = 0; a < D; ++a)
                for (int b = 0; b < D; ++b) fin[b * D + a] = S[a * D + b];
            free(S);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------ decode core */

/*
 * Decode / spec-verify recurrent core (reference.py:155-171), B sequences x S tokens, H heads, on the V-major
 * state st[v][k]:
 *     st *= exp(g)[k];   u[v] = beta (v[v] - sum_k st[v,k] k[k]);   st[v,k] += u[v] k[k];   o[v] = scale sum_k st[v,k] q[k]
 *   q, k, v, g : [B*S, H, 128] (token-major, q/k normalized);  beta: [B*S, H]
 *   S_in       : [B, H, 128, 128] V-major start states
 *   S_steps    : [B, S, H, 128, 128] V-major state after every token (written)
 *   out        : [B*S, H, 128] (written)
 */
#define DEFINE_REC(NAME, REAL, EXP)                                                                            \
    static void NAME(const float* q, const float* k, const float* v, const float* g, const float* beta,       \
                     int S, int H, double scale, const float* sin, float* steps, float* o) {                   \
        REAL* st = (REAL*)malloc(sizeof(REAL) * D * D);                                                        \
        for (int i = 0; i < D * D; ++i) st[i] = sin[i];                                                        \
        const int64_t ts = (int64_t)H * D;                                                                     \
        for (int t = 0; t < S; ++t) {                                                                          \
            const float* qt = q + t * ts; const float* kt = k + t * ts;                                        \
            const float* vt = v + t * ts; const float* gt = g + t * ts;                                        \
            const REAL b = (REAL)beta[(int64_t)t * H];                                                         \
            REAL dec[D];                                                                                       \
            for (int c = 0; c < D; ++c) dec[c] = EXP((REAL)gt[c]);                                             \
            for (int r = 0; r < D; ++r) {                                                                      \
                REAL* row = st + r * D;                                                                        \
                REAL kS = 0;                                                                                   \
                for (int c = 0; c < D; ++c) { row[c] *= dec[c]; kS += row[c] * (REAL)kt[c]; }                  \
                const REAL u = b * ((REAL)vt[r] - kS);                                                         \
                REAL acc = 0;                                                                                  \
                for (int c = 0; c < D; ++c) { row[c] += u * (REAL)kt[c]; acc += row[c] * (REAL)qt[c]; }        \
                o[t * ts + r] = (float)((REAL)scale * acc);                                                    \
            }                                                                                                  \
            float* dst = steps + (int64_t)t * H * D * D;                                                       \
            for (int i = 0; i < D * D; ++i) dst[i] = (float)st[i];                                             \
        }                                                                                                      \
        free(st);                                                                                              \
    }

DEFINE_REC(rec_f32, float, expf)
DEFINE_REC(rec_f64, double, exp)

int kdao_recurrent(const float* q, const float* k, const float* v, const float* g, const float* beta, int B, int S,
                   int H, double scale, const float* S_in, float* S_steps, float* out, int precision, int nthreads) {
    if (B < 0 || S <= 0 || H <= 0 || (precision != 32 && precision != 64)) return -1;
    const int64_t pairs = (int64_t)B * H;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t p = 0; p < pairs; ++p) {
        const int n = (int)(p / H), h = (int)(p % H);
        const int64_t tok = (int64_t)n * S;
        const int64_t off = tok * H * D + (int64_t)h * D;
        const float* sin = S_in + ((int64_t)n * H + h) * D * D;
        /* steps of sequence n, head h: [S, H, 128, 128] block of sequence n, offset by the head */
        float* steps = S_steps + ((int64_t)n * S * H + h) * D * D;
        if (precision == 64)
            rec_f64(q + off, k + off, v + off, g + off, beta + tok * H + h, S, H, scale, sin, steps, out + off);
        else
            rec_f32(q + off, k + off, v + off, g + off, beta + tok * H + h, S, H, scale, sin, steps, out + off);
    }
    return 0;
}

/* Threads the OpenMP runtime would use (reported next to the CPU baseline). */
int kdao_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
