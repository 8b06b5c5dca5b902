/*
 * kda_bt16_hip.h -- C ABI of libkda_bt16_hip.so, the MI355X (gfx950) KDA
 * BT=16 chunked forward.
 *
 * The reference exposes this path only as Python/Triton:
 *   kda_bt16_fwd    /root/reference/src/kda_bt16/kernels.py:752-810
 *   kda_bt16_debug  /root/reference/src/kda_bt16/kernels.py:813-850
 *   _run (host driver, two launches)  kernels.py:475-606
 *   kda_bt16_kernel_k1 (intra-chunk)  kernels.py:53-184
 *   kda_bt16_kernel_k2 (state/output) kernels.py:187-302
 * The entry points below are what a binding of that path calls: device
 * pointers, sizes and flags only, no framework types.  Every call is
 * asynchronous on the caller's HIP stream and returns 0 or a negative
 * KDA_BT16_E* code; nothing is allocated inside the library.
 *
 * Tensor layouts (all row-major, contiguous, on one device):
 *   q, k      [B, T, H, 128]   bf16
 *   v         [B, T, HV, 128]  bf16   HV a multiple of H: value head hv
 *                                     reads q/k head hv / (HV / H)
 *                                     (kernels.py:88; the reference's
 *                                     validation requires HV == H)
 *   g         [B, T, HV, 128]  fp32 or bf16: the raw gate (USE_GATE), the
 *                                     per-token natural-log decay
 *                                     (G_LOG_DECAY), or else the precomputed
 *                                     chunk-local log2 cumsum
 *   beta      [B, T, HV]       fp32 or bf16
 *   A_log     [HV]             fp32
 *   dt_bias   [HV * 128]       fp32 (optional)
 *   h0, ht    [S, HV, 128, 128] fp32, [V, K] if KDA_BT16_STATE_V_FIRST is
 *                              set, else [K, V] (optional); S = B, or N
 *                              with cu_seqlens
 *   o         [B, T, HV, 128]  bf16 (fp32 with KDA_BT16_O_FP32, recurrence only)
 *   cu_seqlens [N + 1]         int32 or int64 (optional): N sequences packed
 *                              along T with B == 1, sequence n holding
 *                              tokens [cu_seqlens[n], cu_seqlens[n+1]),
 *                              cu_seqlens[0] == 0, cu_seqlens[N] == T,
 *                              non-decreasing (FLA's varlen convention; the
 *                              reference lists varlen as a limitation,
 *                              README.md:420-421).  Values outside that
 *                              contract give unspecified results but never
 *                              an access outside the tensors.
 * Debug outputs (optional, reference layouts, kernels.py:572-579):
 *   dbg_Aqk, dbg_A_inv [B, T, HV, 16] bf16; dbg_w, dbg_u [B, T, HV, 128] bf16;
 *   dbg_g [B, T, HV, 128] fp32.
 */
#ifndef KDA_BT16_HIP_H
#define KDA_BT16_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KDA_BT16_ABI_VERSION 4

/* Flags: the reference's tl.constexpr switches (kernels.py:78-82, 208-212).
 * USE_INITIAL_STATE / STORE_FINAL_STATE / HAS_BIAS / STORE_A_INV follow from
 * which pointers are non-NULL and need no flag. */
#define KDA_BT16_USE_GATE          (1u << 0) /* USE_GATE          kernels.py:115 */
#define KDA_BT16_USE_QK_L2NORM     (1u << 1) /* USE_QK_L2NORM     kernels.py:108 */
#define KDA_BT16_USE_BETA_SIGMOID  (1u << 2) /* USE_BETA_SIGMOID  kernels.py:98  */
#define KDA_BT16_STATE_V_FIRST     (1u << 3) /* STATE_V_FIRST     kernels.py:218 */
/* kda_recurrent_fwd_hip only (the chunked entries reject it): o is fp32. */
#define KDA_BT16_O_FP32            (1u << 4)
/* Without USE_GATE: g is the per-token natural-log decay (alpha_t = exp(g_t),
 * FLA's chunk_kda / fused_recurrent_kda convention) and stage 1 forms its
 * chunk-local log2 cumsum, as kda_gate_chunk_cumsum does for the gate
 * (tests/test_kda_bt16.py:16).  No effect with USE_GATE. */
#define KDA_BT16_G_LOG_DECAY       (1u << 5)
/* The forward entries (kda_bt16_fwd_hip, kda_bt16_fwd_noalloc_hip,
 * kda_bt16_fwd_plan): run the fused kernel whatever the (sequence, value
 * head) count, the reference's use_fused_kernel=True (kernels.py:769-810,
 * its single-kernel variant kernels.py:305-472).  Debug outputs still take
 * the two stages; the other entries ignore it. */
#define KDA_BT16_FUSED_KERNEL      (1u << 6)
/* The forward entries: run stage 1 then stage 2 whatever the (sequence,
 * value head) count.  Not with KDA_BT16_FUSED_KERNEL (KDA_BT16_EINVAL). */
#define KDA_BT16_TWO_STAGE         (1u << 7)

/* Element types of g and beta, and of cu_seqlens. */
#define KDA_BT16_DTYPE_F32  0
#define KDA_BT16_DTYPE_BF16 1
#define KDA_BT16_DTYPE_I32  2
#define KDA_BT16_DTYPE_I64  3

/* Error codes. */
#define KDA_BT16_OK                 0
#define KDA_BT16_EINVAL            -1 /* null pointer, non-positive size, bad dtype tag,
                                         misaligned tensor (16 B; beta its element size;
                                         Aqk/A_inv 8 B; cu_seqlens its element size),
                                         cu_seqlens with B != 1 or N <= 0, both
                                         KDA_BT16_FUSED_KERNEL and KDA_BT16_TWO_STAGE,
                                         k2_tiles not 0/1/2/4/8, k2_wave_tiles not 0/1/2,
                                         max_seqlen < 0 */
#define KDA_BT16_EUNSUPPORTED      -2 /* K != 128, V != 128 (kernels.py:727-728) or HV not
                                         a multiple of H; work beyond the 32-bit grids or
                                         per-sequence record sizes (T > 1973776), and
                                         KDA_BT16_O_FP32 on a chunked entry. */
#define KDA_BT16_EWORKSPACE        -3 /* workspace missing or smaller than kda_bt16_workspace_bytes */
#define KDA_BT16_ELAUNCH           -4 /* HIP launch error */
#define KDA_BT16_EABI              -5 /* args->abi_version != KDA_BT16_ABI_VERSION */
#define KDA_BT16_ERANGE            -6 /* lower_bound outside (-11, 0) with USE_GATE (kernels.py:733-744) */
#define KDA_BT16_ESCRATCH          -7 /* kda_bt16_fwd_noalloc_hip: the geometry needs more than
                                         KDA_BT16_NOALLOC_MAX_WORKSPACE bytes of records,
                                         even in chunk ranges */

/* Size of the static device scratch of kda_bt16_fwd_noalloc_hip (96 MiB:
 * 5782 records of 17 KiB, e.g. B=2 T=4096 H=8, or 92.5k tokens of one
 * value head). */
#define KDA_BT16_NOALLOC_MAX_WORKSPACE ((size_t)96 << 20)

typedef struct KdaBt16Args {
    int32_t abi_version; /* KDA_BT16_ABI_VERSION */
    int32_t B, T, H, HV, K, V;
    uint32_t flags;      /* KDA_BT16_* flag bits */
    float scale;         /* already resolved: the API substitutes K**-0.5 for None */
    float lower_bound;
    int32_t g_dtype;     /* KDA_BT16_DTYPE_* */
    int32_t beta_dtype;  /* KDA_BT16_DTYPE_* */
    const void* q;
    const void* k;
    const void* v;
    const void* g;
    const void* beta;
    const float* A_log;   /* required with USE_GATE */
    const float* dt_bias; /* optional */
    const float* h0;      /* optional initial state */
    void* o;              /* required */
    float* ht;            /* optional final state */
    void* workspace;      /* kda_bt16_workspace_bytes() bytes, 256-byte aligned; not read
                             (may be NULL) when the forward runs fused */
    size_t workspace_bytes;
    void* dbg_Aqk;        /* optional debug outputs, all or none */
    void* dbg_A_inv;
    void* dbg_w;
    void* dbg_u;
    float* dbg_g;
    const void* cu_seqlens;   /* optional: packed sequences (varlen) */
    int32_t cu_seqlens_dtype; /* KDA_BT16_DTYPE_I32 or KDA_BT16_DTYPE_I64 */
    int32_t N;                /* number of sequences with cu_seqlens */
    /* The forward's kernel choices (ABI 4).  Each 0 leaves the choice to
     * the library; every choice gives the same results bit for bit. */
    int32_t k2_tiles;         /* stage-2 value tiles per work-group: 1, 2, 4 or 8 */
    int32_t k2_wave_tiles;    /* with 2-8 tiles per work-group, 1 or 2 forces compute waves
                                 of that many whole tiles (0: a state wave per tile at 2
                                 tiles, two-tile compute waves at 8, one-tile at 4) */
    int32_t max_seqlen;       /* with cu_seqlens: the longest sequence's length, when the
                                 caller knows it (a hint for the choice between the fused
                                 kernel and the two stages; a wrong value changes only the
                                 choice, never the results) */
} KdaBt16Args;

/* Bytes of scratch the two stages exchange for a fixed-length geometry (one
 * 17 KiB record per (batch, value head, 16-token chunk)).  Replaces the
 * reference's intermediate allocations Aqk / Akk_scratch / w / u / g_cumsum,
 * kernels.py:572-579.  Returns 0 for an unsupported geometry. */
size_t kda_bt16_workspace_bytes(int32_t B, int32_t T, int32_t HV, int32_t K, int32_t V);

/* The same for any arguments, varlen included (HV * (floor(T/16) + N)
 * records with cu_seqlens).  Reads only the size fields and cu_seqlens'
 * presence, never the device memory. */
size_t kda_bt16_workspace_bytes_args(const KdaBt16Args* args);

/* Full forward on `stream` (a hipStream_t; NULL is the legacy default
 * stream).  Replaces _run's two launches, kernels.py:581-602: stage 1 then
 * stage 2 (kda_bt16_k1_hip, kda_bt16_k2_hip), or one fused kernel that
 * keeps stage 1's per-chunk records in LDS instead of the workspace (same
 * results bit for bit).  The choice (kda_bt16_fwd_plan) depends on the
 * arguments and the device's CU count only:
 *   - debug outputs: the two stages;
 *   - KDA_BT16_FUSED_KERNEL: fused; KDA_BT16_TWO_STAGE: the two stages;
 *   - fixed length: fused when the (batch row, value head) pairs are more
 *     than half the CUs;
 *   - cu_seqlens without max_seqlen: fused when the pairs are at least as
 *     many as the CUs;
 *   - cu_seqlens with max_seqlen: fused when its estimated time (set by the
 *     longest sequence's chunks, or by the chunks per CU) is at most the two
 *     stages' (set by all chunks for stage 1 and the longest chain for
 *     stage 2), so one long sequence among short ones keeps the two stages.
 * The workspace is required when the call runs the two stages and ignored
 * (may be NULL) when it runs fused. */
int kda_bt16_fwd_hip(const KdaBt16Args* args, void* stream);

/* Which kernels kda_bt16_fwd_hip (and kda_bt16_fwd_noalloc_hip) run for
 * these arguments on the current device: 1 the fused kernel, 0 stage 1 then
 * stage 2, or a negative KDA_BT16_E* code for invalid arguments.  Reads no
 * device memory and needs no workspace.  No counterpart in the reference,
 * whose _run always launches its two stages (kernels.py:581-602). */
int kda_bt16_fwd_plan(const KdaBt16Args* args);

/* In how many segments of consecutive chunks kda_bt16_fwd_hip runs its two
 * stages for these arguments on the current device: 0 when it runs fused,
 * else 1 to 64, or a negative KDA_BT16_E* code for invalid arguments.  A
 * fixed-length forward with more than 200 MB of records runs stage 1 then
 * stage 2 on each range of about 150 MB of records in turn, stage 2
 * carrying the state across (results bit for bit those of one pass); every
 * segment's records and the state between them fit the workspace of
 * kda_bt16_workspace_bytes_args.  Reads no device memory.  No counterpart
 * in the reference; for measurement (the stage-level entry points run one
 * pass). */
int kda_bt16_fwd_segments(const KdaBt16Args* args);

/* Work-groups of the fused kernel that gave up a wait on the current
 * device since the library was loaded or the count last reset.  No
 * counterpart in the reference.  The fused kernel's waves meet through LDS
 * flags, and every wait is bounded (2^22 polls) so that a stalled
 * work-group cannot hang the GPU; one that runs out writes NaN over the o
 * columns and final-state rows of its compute waves that had not finished
 * (a wave that finished first consumed only completed chunks) and adds 1
 * to this count.  Synchronous: it waits for the device's work to finish.  With
 * `reset` non-zero the count is set back to 0 after it is read.  Not for
 * use during graph capture. */
int kda_bt16_fused_aborts(uint32_t* count, int32_t reset);

/* Full forward that allocates nothing and takes no workspace.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The same kernels as kda_bt16_fwd_hip,
 * with the same results bit for bit.
 *   - When the forward runs fused (kda_bt16_fwd_plan) it uses no scratch
 *     and takes any size.
 *   - Otherwise the records stage 1 hands to stage 2 live in a file-scope
 *     device array of KDA_BT16_NOALLOC_MAX_WORKSPACE bytes.  A fixed-length
 *     geometry whose records do not fit runs its two stages in consecutive
 *     chunk ranges short enough to fit, with the state between them in the
 *     array too (B=1 T=8192 H=32: 3 ranges of 170-171 chunks); packed
 *     sequences, debug outputs, or so many (row, value head) pairs that not
 *     even one-chunk ranges fit, return KDA_BT16_ESCRATCH before any
 *     launch.  The first such call on a device looks up the
 *     array's device address (the runtime places the array on that device
 *     then, and the library holds it until the process ends): make that
 *     first call before capturing calls into a graph.
 *   - Every call on one GPU uses that GPU's one array: calls that overlap
 *     on one GPU (two streams, two threads) race and give wrong results;
 *     calls in order on one stream are safe.  The array keeps the last
 *     call's contents; no part of it needs clearing (stage 1 writes every
 *     record stage 2 reads).
 * args->workspace and args->workspace_bytes are ignored. */
int kda_bt16_fwd_noalloc_hip(const KdaBt16Args* args, void* stream);

/* Stage 1 only: per-chunk gates, grams, (I+L)^-1 solve and W/U into the
 * workspace, plus the debug outputs when given.  Replaces the
 * kda_bt16_kernel_k1 launch, kernels.py:581-592. */
int kda_bt16_k1_hip(const KdaBt16Args* args, void* stream);

/* Stage 2 only: the serial state recurrence over the records stage 1 wrote;
 * writes o and ht.  Replaces the kda_bt16_kernel_k2 launch,
 * kernels.py:593-602. */
int kda_bt16_k2_hip(const KdaBt16Args* args, void* stream);

/* Token-by-token recurrence in fp32 on `stream`: the decode step (T = 1)
 * and the fused-recurrent forward for any T.  No counterpart in the
 * reference, whose roadmap lists the decode step (README.md:503-505) and
 * whose tests use FLA's fused_recurrent_kda as gold
 * (tests/test_kda_bt16.py:26-38); same arguments as that call.
 * Same layouts, flags and g conventions as the chunked entries, varlen and
 * grouped value heads included.  Differences:
 *   - o is fp32 with KDA_BT16_O_FP32, else bf16;
 *   - no workspace and no debug outputs (workspace fields are ignored, the
 *     debug pointers must be NULL);
 *   - h0 and ht may be the same buffer (the state updated in place). */
int kda_recurrent_fwd_hip(const KdaBt16Args* args, void* stream);

/* Backward of the chunked forward (no counterpart in the reference, which is
 * forward-only, README.md:420; its training graph is FLA's chunk_kda_bwd,
 * docs/KDA_ANALYSIS.md:134-165).  Gradients of sum(o * dO) + sum(ht * dht)
 * with respect to every input, for the same arguments as the forward:
 * recompute (stage 1, stage 2 storing the per-chunk states), the reverse
 * state-gradient chain, the per-chunk gradients, and the gate-parameter
 * sums.  Asynchronous on `stream`; allocates nothing. */
typedef struct KdaBt16BwdArgs {
    const KdaBt16Args* fwd; /* the forward's arguments: inputs, sizes, flags,
                               cu_seqlens; its o, ht, workspace and debug
                               pointers are ignored (debug must be NULL) */
    const void* dout;       /* dO [B, T, HV, 128] bf16, required */
    const float* dht;       /* optional gradient of ht (state layout of the flags) */
    void* dq;               /* [B, T, H, 128] bf16, required */
    void* dk;               /* [B, T, H, 128] bf16, required */
    void* dv;               /* [B, T, HV, 128] bf16, required */
    void* dg;               /* shape and element type of g, required */
    void* dbeta;            /* shape and element type of beta, required */
    float* dA_log;          /* optional [HV]; only with USE_GATE */
    float* ddt_bias;        /* optional [HV * 128]; only with USE_GATE and dt_bias */
    float* dh0;             /* optional gradient of the initial state (its layout) */
    void* workspace;        /* kda_bt16_bwd_workspace_bytes() bytes, 256-byte aligned */
    size_t workspace_bytes;
} KdaBt16BwdArgs;

/* Workspace of kda_bt16_bwd_hip: per 16-token record slot, the forward and
 * the backward records (17 KiB each), bf16 h and dh (32 KiB each), v_new and
 * dv_new (4 KiB each) and the gate partial sums (528 B): ~106.5 KiB
 * (1.70 GiB at B=1 T=8192 H=32).  Returns 0 for an unsupported geometry. */
size_t kda_bt16_bwd_workspace_bytes(const KdaBt16Args* fwd);

int kda_bt16_bwd_hip(const KdaBt16BwdArgs* args, void* stream);

/* Training forward that keeps its state for the backward (no counterpart in
 * the reference, which is forward-only; FLA's chunk_kda forward saves its
 * per-chunk states the same way, docs/KDA_ANALYSIS.md:134-165).  o and ht as
 * kda_bt16_fwd_hip, bit for bit (args->workspace as there), and into `saved`
 * (kda_bt16_saved_bytes(args) bytes, 256-byte aligned) what the backward
 * would otherwise recompute: per 16-token record slot the backward record
 * without dO (17 KiB), bf16 h (32 KiB), v_new (4 KiB) and the gram block
 * (2 KiB), ~55 KiB (880 MiB at B=1 T=8192 H=32).  No debug outputs.
 * Asynchronous on `stream`; allocates nothing. */
size_t kda_bt16_saved_bytes(const KdaBt16Args* fwd);

int kda_bt16_fwd_save_hip(const KdaBt16Args* args, void* saved, size_t saved_bytes, void* stream);

/* Backward from the state kda_bt16_fwd_save_hip kept (same forward
 * arguments): the gradients of kda_bt16_bwd_hip, bit for bit, without its
 * recompute.  args->workspace: kda_bt16_bwd_saved_workspace_bytes() bytes
 * (dh, dv_new, gate partial sums; ~36.5 KiB per slot).  dO is written into
 * the saved backward records, so the saved state may serve several
 * backward calls but not two at once. */
size_t kda_bt16_bwd_saved_workspace_bytes(const KdaBt16Args* fwd);

int kda_bt16_bwd_saved_hip(const KdaBt16BwdArgs* args, void* saved, size_t saved_bytes, void* stream);

/* Static message for an error code. */
const char* kda_bt16_strerror(int code);

/* KDA_BT16_ABI_VERSION of the built library. */
int kda_bt16_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* KDA_BT16_HIP_H */
