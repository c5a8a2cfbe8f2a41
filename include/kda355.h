/*
 * kda355.h -- C ABI of the MI355X (gfx950) KDA library libkda355.so.
 *
 * KDA (Kimi Delta Attention): the gated delta rule with a per-key-channel decay, head dim K = V = 128, fp32
 * state stored V-major [V][K] (128 x 128 floats = 64 KiB per (sequence, head)).
 *
 * Every entry point takes a POD argument struct of raw device pointers, element strides and sizes plus a
 * hipStream_t, launches asynchronously on that stream and returns a status code.  Nothing here allocates device
 * memory, synchronizes, or keeps per-call global state, so every launch entry point is safe inside HIP-graph
 * capture and re-entrant across threads and streams.  bf16 / fp16 tensors are passed as `const void*`.
 *
 * Status codes: 0 = launched; KDA355_EINVAL (-1) = invalid arguments (nothing launched, kda355_last_error()
 * names the argument); KDA355_ELAUNCH (-2) = the HIP launch failed.
 *
 * Which reference interface each entry point replaces (caoshiyi/eat-kernels paths):
 *   kda355_recurrent_launch       vLLM fused_recurrent_kda as called by the Kimi layer
 *                                 (kda/mi350x/benchmark/vllm_reference/kda.py:488-502, 560-575) and the recurrent
 *                                 core of the decode kernel's `run` binding (kda/mi350x/kda/decode/kda_v14_b.cu:
 *                                 3266-3312, slot rules `slots()` :1013-1042)
 *   kda355_decode_launch          the fused decode / spec-verify step of the vLLM-ROCm Kimi layer, `decode(mixed_qkv,
 *                                 conv_state, ...)` (kda/mi350x/kda/kernel.py:212-216; semantics
 *                                 kda/mi350x/reference.py:104-181; input contract kda/mi350x/kda/decode/kernel_v13_a.py:
 *                                 697-735; slot rules kda/mi350x/kda/decode/kda_v14_b.cu:1013-1042)
 *   kda355_spec_commit_launch     the commit of an accepted draft length (kda/mi350x/reference.py:117-121 reads the
 *                                 state after token a-1; this copies it to the sequence's pool slot)
 *   kda355_prefill_plan           kda_build_meta (kda/mi350x/kda/prefill/kernel.h:100-102) and prepare_prod
 *                                 (kda/mi350x/kda/prefill/main.cpp:103-130): host-only schedule tables
 *   kda355_prefill_workspace_bytes  kda_workspace_floats (kda/mi350x/kda/prefill/kernel.h:90-91)
 *   kda355_prefill_launch         kda_prefill_kernel_launch (kda/mi350x/kda/prefill/kernel.h:33-56) with the
 *                                 KdaPool production contract (kernel.h:19-31)
 */
#ifndef KDA355_H
#define KDA355_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* kda355_stream_t; /* == hipStream_t */

#define KDA355_EINVAL (-1)
#define KDA355_ELAUNCH (-2)
#define KDA355_HEAD_DIM 128
#define KDA355_CHUNK 64
/* Smallest per-token log-decay the chunked prefill uses: its diagonal Gram blocks hold e^{+-8 g} over 8 tokens, which
   for g >= -9 stays inside 2^{+-104}, where fp32 and bf16 are normal with room for the low half of a bf16 pair (the
   MFMAs flush subnormal operands).  A log-decay below it (given, or formed in the kernel from a lower_bound below it)
   is raised to it, which changes the state by less than e^{-9} = 1.2e-4 of the affected channel.  The
   reference guards the same range by recomputing overflowed slices in fp32 (kda/mi350x/kda/kernel.py:113-128). */
#define KDA355_MIN_LOG_DECAY (-9.0f)

/* ------------------------------------------------------------------------------------------------ recurrent */

/* flags of KdaRecurrentArgs */
#define KDA355_REC_NORMALIZE_QK 1u  /* q, k <- x * rsqrt(sum x^2 + 1e-6) in the kernel (kda/mi350x/reference.py:159-160) */
#define KDA355_REC_RAW_GATE 2u      /* g is bf16 raw_g: g = lower_bound * sigmoid(exp(A_log[h]) * (raw_g + dt_bias[h,k])) */
#define KDA355_REC_RAW_BETA 4u      /* beta is bf16 raw_beta: beta = sigmoid(raw_beta) */
#define KDA355_REC_PER_TOKEN 8u     /* write the state after every token t to write_idx[n, t] (spec verify);
                                       otherwise the final state goes back to the read row (plain decode) */
#define KDA355_REC_SLOT0_RESERVED 16u /* row 0 of read_pool is the padding slot: never read, never written */
#define KDA355_REC_WRITE_SLOT0_RESERVED 32u /* the same rule for write_pool (PER_TOKEN destinations) */

/*
 * Recurrent decode / speculative verify over B sequences x S tokens (T = B*S rows, row n*S + t is token t of
 * sequence n), H heads.  Per (n, h):
 *     read row   r = read_idx[n * read_idx_stride + (num_accepted ? clamp(num_accepted[n], 1, S) - 1 : 0)]
 *     S0         = read_pool[r]      (a padding row -- outside [0, read_slots), or 0 with SLOT0_RESERVED -- is
 *                                     never read; the sequence is skipped and its output rows are zero)
 *     per token: S *= exp(g_t) (key axis);  u = beta_t (v_t - S k_t);  S += u k_t^T;  o_t = scale * S q_t
 *     writes     PER_TOKEN: write_pool[write_idx[n*S + t]] = state after token t (padding rows skipped);
 *                otherwise read_pool[r] = final state.
 * The reference's spec-verify mapping (kda/mi350x/reference.py:135-143,168-171) is read_pool == write_pool,
 * read_idx == write_idx == state_indices [B, S], read_idx_stride = S, num_accepted given, PER_TOKEN.
 */
typedef struct KdaRecurrentArgs {
    const void* q;              /* bf16 [T, H, 128], row stride qkv_row_stride elements */
    const void* k;
    const void* v;
    const void* g;              /* fp32 [T, H, 128] log-decay, or bf16 raw_g with RAW_GATE; row stride g_row_stride */
    const void* beta;           /* fp32 [T, H] activated, or bf16 raw_beta with RAW_BETA; row stride beta_row_stride */
    const float* A_log;         /* [H]        (RAW_GATE only) */
    const float* dt_bias;       /* [H * 128]  (RAW_GATE only) */
    float* read_pool;           /* [read_slots, H, 128, 128] fp32 V-major, slot stride read_slot_stride floats */
    float* write_pool;          /* PER_TOKEN destination pool (may equal read_pool) */
    const int32_t* read_idx;    /* [B, read_idx_stride] */
    const int32_t* num_accepted;/* [B] or NULL */
    const int32_t* write_idx;   /* [B, S] (PER_TOKEN) or NULL */
    void* out;                  /* bf16 [T, H, 128], row stride out_row_stride elements */
    int64_t qkv_row_stride, g_row_stride, beta_row_stride, out_row_stride;
    int64_t read_slot_stride, read_slots, write_slot_stride, write_slots;
    int32_t B, S, H, read_idx_stride;
    float scale, lower_bound;
    uint32_t flags;
    int32_t reserved;
} KdaRecurrentArgs;

int kda355_recurrent_launch(const KdaRecurrentArgs* args, kda355_stream_t stream);

/*
 * Commit of an accepted draft length: for each sequence n with a = clamp(num_accepted[n], 1, S),
 * pool[pool_idx[n]] = scratch[scratch_idx[n*S + a - 1]] (all H heads; padding rows skipped as above).
 */
typedef struct KdaSpecCommitArgs {
    const float* scratch;       /* [scratch_slots, H, 128, 128] */
    float* pool;                /* [pool_slots, H, 128, 128] */
    const int32_t* scratch_idx; /* [B, S] */
    const int32_t* pool_idx;    /* [B] */
    const int32_t* num_accepted;/* [B] */
    int64_t scratch_slot_stride, scratch_slots, pool_slot_stride, pool_slots;
    int32_t B, S, H;
    uint32_t flags;             /* KDA355_REC_SLOT0_RESERVED applies to the pool (scratch rows may use 0) */
} KdaSpecCommitArgs;

int kda355_spec_commit_launch(const KdaSpecCommitArgs* args, kda355_stream_t stream);

/* ------------------------------------------------------------------------------------------------ fused decode */

/*
 * Fused decode / speculative verify of B sequences x S tokens (T = B*S rows, row n*S + t is token t of sequence n),
 * H heads, dim = H * 128, per (n, h) and token t:
 *     conv      x = SiLU(sum_j window[t + j] * conv_weight[:, j]) over the head's q | k | v channels, where window =
 *               3 history taps of conv_state[cs] followed by the S rows of mixed_qkv (width-4 causal depthwise conv)
 *     q, k      x * rsqrt(sum x^2 + 1e-6);  q *= 128^-1/2
 *     gate      g = lower_bound * sigmoid(exp(A_log[h]) * (gate + dt_bias));  beta = sigmoid(beta)
 *     rule      S *= exp(g) (key axis);  u = beta (v - S k);  S += u k^T;  o = S q
 *     output    y = bf16(o) * rsqrt(mean(bf16(o)^2) + norm_eps) * norm_weight * sigmoid(out_gate)   (bf16)
 * plain decode (num_accepted == NULL, state_indices [B]): rd = cs = state_indices[n]; the final state goes back to
 *     ssm_state[rd]; conv_state[cs] taps [0, 3) <- the last 3 window rows (taps beyond 3 are untouched).
 * spec verify (num_accepted [B], state_indices [B, S]): a = clamp(num_accepted[n], 1, S), rd = state_indices[n, a-1],
 *     cs = state_indices[n, 0]; history taps [a-1, a+2); the state after token t goes to ssm_state[state_indices[n, t]]
 *     (rows <= 0 skipped); conv_state[cs] taps [0, 2 + S) <- window rows [1, 3 + S).
 * Rows <= 0 or outside the pool are padding: a sequence whose rd or cs is padding gets zero output rows and writes
 * nothing.  The vLLM page layout (conv_state and ssm_state as strided views into one byte pool) is expressed by the
 * slot strides.  S <= 16.
 */
typedef struct KdaDecodeArgs {
    const void* mixed_qkv;      /* bf16 [T, 3 * dim], row stride mixed_row_stride elements (16-byte aligned rows) */
    void* conv_state;           /* bf16 [conv_slots, conv_taps, 3 * dim]: slot / tap strides in elements */
    const float* conv_weight;   /* [3, 4, dim] dense: (q | k | v, tap, channel) */
    const void* gate;           /* bf16 [T, H, 128], row stride gate_row_stride elements */
    const void* beta;           /* bf16 [T, H] logits, row stride beta_row_stride */
    const void* out_gate;       /* bf16 [T, dim], row stride out_gate_row_stride */
    const float* A_log;         /* [H] */
    const float* dt_bias;       /* [dim] */
    const float* norm_weight;   /* [128] */
    float* ssm_state;           /* [ssm_slots, H, 128, 128] fp32 V-major, slot stride ssm_slot_stride floats */
    const int32_t* state_indices;  /* [B] (plain) or [B, S] (spec), dense */
    const int32_t* num_accepted;   /* [B] or NULL (plain decode) */
    void* out;                  /* bf16 [T, dim], row stride out_row_stride */
    int64_t mixed_row_stride, gate_row_stride, beta_row_stride, out_gate_row_stride, out_row_stride;
    int64_t conv_slot_stride, conv_tap_stride, conv_slots, ssm_slot_stride, ssm_slots;
    int32_t B, S, H, conv_taps;
    float norm_eps, lower_bound;
    uint32_t flags;             /* 0 */
    int32_t reserved;
    void* workspace;            /* NULL, or KDA355_DECODE_WS_BYTES of device memory whose first 256 bytes (the
                                   counters) are zero before the first launch: launches of at most 64 (sequence, head)
                                   pairs (B * H) then split each state over 4 workgroups, the last of which finishes the
                                   head's outputs.  Each such launch leaves the counters zero again (the rest is
                                   written before it is read); launches that may run at the same time on one GPU need
                                   workspaces of their own.  No counterpart in the reference's decode entry (its
                                   single-launch small-batch kernel is kda/mi350x/kda/decode/kda_v14_b.cu:1856-). */
} KdaDecodeArgs;

/* Bytes of the decode workspace: 64 int32 counters, then 64 x 4 x 16 fp32 partial sums of squares. */
#define KDA355_DECODE_WS_BYTES 16640

int kda355_decode_launch(const KdaDecodeArgs* args, kda355_stream_t stream);

/* ------------------------------------------------------------------------------------------------ prefill */

/* flags of KdaPrefillPlanIn / KdaPrefillArgs */
#define KDA355_PF_NORMALIZE_QK 1u  /* q, k <- x / max(|x|, 1e-6) in the kernel (kda/mi350x/reference.py:59-60) */
#define KDA355_PF_RAW_GATE 2u      /* g is bf16 raw_g: g = lower_bound * sigmoid(exp(A_log[h]) * (raw_g + dt_bias[h,k])) */
#define KDA355_PF_RAW_BETA 4u      /* beta is bf16 raw_beta (any row stride): beta = sigmoid(raw_beta) */
#define KDA355_PF_POOL 8u          /* states live in a paged pool: read state_pool[state_idx[n]] when has_initial_state[n]
                                      (else start from zero and never read the row), write the final state there */
#define KDA355_PF_CK_SINGLE 16u    /* one checkpoint per sequence: the state after ck_offsets[n] tokens (a positive
                                      multiple of 64, <= the length; planned on the host) goes to ck_pool[ck_idx[n]]
                                      when ck_idx[n] >= 0 (kda/mi350x/reference.py:38-41,52-57) */
#define KDA355_PF_CK_EVERY 32u     /* every-n checkpoints: row j of sequence n (j < ceil(len_n / ck_every)) is the state
                                      before token j * ck_every, stored to ck_pool[ck_idx[row_start_n + j]] with
                                      row_start_n = sum of the earlier sequences' row counts (kda/b200/kda_b200.py:19-22) */
#define KDA355_PF_PRECISE 64u      /* the solve's and the state update's fp16 operands as fp16 pairs (22 bits): about half
                                      the state error on chunks of nearly parallel keys with beta ~ 1, ~11 % more time.
                                      No counterpart in the reference (its prefill precision is fixed). */
#define KDA355_PF_CHUNK64 128u     /* keep the 64-token kernel (and the plan's workgroup lists) where the plan chose the
                                      32-token kernel (KdaPrefillPlan.chunk32); a comparison and test switch.  No
                                      counterpart in the reference. */

/* Host-side plan input: the layout only (never the data). */
typedef struct KdaPrefillPlanIn {
    const int64_t* cu_seqlens;  /* host [N + 1] token offsets */
    const int32_t* ck_offsets;  /* host [N] single-checkpoint offsets (tokens) or NULL */
    int32_t N, H;
    int32_t ck_every;           /* every-n interval in tokens (multiple of 64) or 0 */
    int32_t num_cus;            /* CUs of the device (0: 256); long sequences are split into pieces of >= 16 chunks
                                   when that shortens the schedule (the chains alone would leave CUs idle, or the
                                   longest ones would finish well after the rest) */
    uint32_t flags;             /* unused (0): checkpoint work is scheduled for every kind the layout defines */
    int32_t reserved;
} KdaPrefillPlanIn;

/* Filled by kda355_prefill_plan. */
typedef struct KdaPrefillPlan {
    int64_t T;
    int32_t N, H, num_chunks, num_chains, max_chain_chunks, ck_every;
    int64_t table_words;        /* int32 words of the schedule table (copy it to the device once per layout) */
    int64_t workspace_bytes;    /* device workspace the launch needs (256-byte aligned) */
    int64_t ck_rows;            /* every-n rows the layout writes (sum over n of ceil(len_n / ck_every)) */
    uint32_t magic, flags;
    int32_t num_pieces;         /* pieces of split sequences (0: no sequence is split) */
    int32_t num_split;          /* split sequences */
    int32_t num_fix_tasks;      /* groups of <= 2 chunks of the later pieces of split sequences (outputs completed after
                                   the scan) */
    int32_t num_ck_tasks;       /* checkpoints inside later pieces (composed after the scan) */
    int32_t chunk_grid;         /* workgroups of the chunk launch: 0 = one per (chain, head); > 0 (layouts without
                                   split sequences whose (chain, head) pairs outnumber the CUs) = that many
                                   workgroups, each walking a list of (chain, head) pairs in turn */
    int32_t chunk32;            /* 1: the launch runs the 32-token chunk kernel, one workgroup per (chain, head) and two
                                   per CU (layouts without split sequences whose items outnumber the CUs, when its
                                   simulated schedule beats chunk_grid's); launches with KDA355_PF_PRECISE or
                                   KDA355_PF_CHUNK64 keep the 64-token kernel.  May be set to 1 by the caller for any
                                   plan without split sequences. */
} KdaPrefillPlan;

/*
 * Schedule of one batch layout (host only, no device call).  Call once with tables == NULL to get
 * plan->table_words, then with a host buffer of that many int32 words, and copy the buffer to the device.
 */
int kda355_prefill_plan(const KdaPrefillPlanIn* in, KdaPrefillPlan* plan, int32_t* tables, int64_t capacity);
int64_t kda355_prefill_workspace_bytes(const KdaPrefillPlan* plan);

/*
 * Chunked prefill over a packed varlen batch (T tokens, N sequences, H heads):
 *   q, k, v [T, H, 128] bf16; g [T, H, 128] fp32 log-decay or bf16 raw gate; beta [T, H] fp32 or bf16 raw;
 *   out [T, H, 128] bf16.  Per (n, h) the token recurrence of kda/mi350x/reference.py:85-91 with scale.
 * States: KDA355_PF_POOL -> state_pool [state_slots, H, 128, 128] (rows dense, slot stride state_slot_stride floats),
 * else initial_state [N, H, 128, 128] (NULL = zeros) and final_state [N, H, 128, 128], contiguous.
 * Checkpoint rows go to ck_pool (fp32, or bf16 rounded to nearest even when ck_dtype == 1), slot stride in elements.
 * Rows outside [0, slots) are skipped.  Asynchronous on `stream`; no host synchronization.
 */
typedef struct KdaPrefillArgs {
    const void* q;
    const void* k;
    const void* v;
    const void* g;
    const void* beta;
    const float* A_log;
    const float* dt_bias;
    void* out;
    float* state_pool;
    const int32_t* state_idx;        /* [N] */
    const uint8_t* has_initial_state;/* [N] bool */
    const float* initial_state;
    float* final_state;
    void* ck_pool;
    const int32_t* ck_idx;           /* CK_SINGLE: [N] rows; CK_EVERY: [ck_rows] rows */
    const int32_t* tables;           /* device copy of the plan's schedule table */
    void* workspace;                 /* >= plan->workspace_bytes, 256-byte aligned */
    int64_t qkv_row_stride, g_row_stride, beta_row_stride, out_row_stride;  /* elements between tokens, each
                                                                              in [0, 2^21) */
    int64_t state_slot_stride, state_slots, ck_slot_stride, ck_slots;
    int64_t T;
    int32_t N, H;
    float scale, lower_bound;
    uint32_t flags;
    int32_t ck_dtype;                /* 0 fp32, 1 bf16 */
    const KdaPrefillPlan* plan;
} KdaPrefillArgs;

int kda355_prefill_launch(const KdaPrefillArgs* args, kda355_stream_t stream);

/*
 * kda355_prefill_launch without a caller workspace.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under graph capture with no allocator at hand, tight serving loops, harnesses that
 * forbid allocation).  args->workspace must be NULL; the workspace of split layouts comes from a static device array
 * of KDA355_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds until the process ends, and a plan whose
 * workspace_bytes exceeds it is rejected with KDA355_EINVAL (config-2-sized layouts need ~1 GB: use
 * kda355_prefill_launch there).  The call allocates nothing.  Calls that overlap on one GPU share the array and
 * race: serialize them (one stream).  Nothing in the array has to start at zero.
 */
#define KDA355_NOALLOC_SCRATCH_BYTES (256ull << 20)
int kda355_prefill_launch_noalloc(const KdaPrefillArgs* args, kda355_stream_t stream);

/* ------------------------------------------------------------------------------------------------ misc */

/* Human-readable reason of the last KDA355_EINVAL / KDA355_ELAUNCH on the calling thread ("" if none). */
const char* kda355_last_error(void);
/* Library version (major * 10000 + minor * 100 + patch). */
int kda355_version(void);

#ifdef __cplusplus
}
#endif

#endif /* KDA355_H */
