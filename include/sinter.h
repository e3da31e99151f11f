/*
 * sinter-mi355x C ABI.
 *
 * The drop-in boundary for the batch-1 decode hot path of a Qwen3.6-27B-shaped
 * hybrid (gated-DeltaNet + full-attention) model on one MI355X (gfx950).  Every
 * entry point is extern "C" with plain pointers and sizes; device pointers are
 * hipMalloc'd memory on the handle's device; no exception crosses the ABI.
 * Functions return SINTER_OK (0) or a negative sinter_status; the message of
 * the last failure on the calling thread is sinter_last_error().
 *
 * Layers (each cites the reference interface it replaces):
 *   1. ISA: sinter_instr and the op payloads -- core/isa.cuh:32-88 and the
 *      per-op Args structs of k0/ops/{gemv,gdn,attn,glue}.cuh.
 *   2. Host control plane: sinter_host_* -- mk::host_* in core/host.h:62-80.
 *   3. Op entry points: sinter_op_* -- one interpreter instruction run as a
 *      standalone launch, the role of the mk_run test wrappers
 *      (tests/test_gemv.cu:57-78, test_gdn.cu:52-83, test_attn.cu:68-98).
 *   4. Model: sinter_model_* -- the harness residency/packer/driver
 *      (k0/harness.cpp:315-566, 1019-1060, 1197-1275) with the schedule
 *      compiler (k0/compile_schedule.py) re-derived for this layout.
 */
#ifndef SINTER_H
#define SINTER_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SINTER_ABI_VERSION 1

/* ------------------------------------------------------------------ status */
enum sinter_status {
    SINTER_OK = 0,
    SINTER_ERR_ARG = -1,     /* bad argument / shape the kernels do not support */
    SINTER_ERR_HIP = -2,     /* HIP runtime call failed */
    SINTER_ERR_DEVICE = -3,  /* device error cell set (see sinter_host_error) */
    SINTER_ERR_TIMEOUT = -4, /* watchdog fired */
    SINTER_ERR_STATE = -5,   /* call out of lifecycle order */
    SINTER_ERR_NOMEM = -6
};
/* core/host.h:31-35 RunStatus */
enum sinter_run_status { SINTER_RUN_OK = 0, SINTER_RUN_ERR = 1, SINTER_RUN_TIMEOUT = 2 };
/* core/interp.cuh:49-56 ErrCode (+ codes of the fused ops) */
enum sinter_err_code {
    SINTER_E_NONE = 0,
    SINTER_E_BAD_KIND = 1,        /* kind >= SINTER_OP_KIND_COUNT */
    SINTER_E_UNWIRED_KIND = 2,    /* valid kind without an implementation */
    SINTER_E_BAD_SHAPE = 3,       /* an op found its payload inconsistent */
    /* 4 is unused: the split-K merge waits on per-chunk generation flags, so
       a partial that was never written is a flag wait that times out (5) */
    SINTER_E_TIMEOUT_BARRIER = 5  /* a grid-barrier or merge-flag wait exceeded the spin limit */
};

const char *sinter_last_error(void);
int sinter_abi_version(void);
/* rig precheck (tests/devinfo.cu): a one-line report of runtime, device and
 * interpreter envelope into buf; non-zero if the device cannot run it */
int sinter_device_info(int device, char *buf, size_t n);

/* ------------------------------------------------------------------ types */
/* ggml_type numbering */
enum sinter_type {
    SINTER_F32 = 0, SINTER_F16 = 1, SINTER_Q8_0 = 8, SINTER_Q4_K = 12,
    SINTER_Q6_K = 14, SINTER_Q8_K = 15, SINTER_BF16 = 30
};
size_t sinter_row_bytes(int type, int64_t k);

/* ------------------------------------------------------------------ ISA */
/* core/isa.cuh:32-81, re-sized: 256-byte instructions (payload 240 B) so the
 * fused ops carry their operands inline; block ranges cover up to 65535
 * workgroups.  Instructions between two BOUNDARY instructions run
 * concurrently on disjoint [block_lo, block_hi) ranges. */
enum sinter_op_kind {
    SINTER_OP_NOP = 0,
    SINTER_OP_BOUNDARY = 1,    /* grid barrier */
    SINTER_OP_GEMV = 2,        /* prologue (norm/embed) + act. quant + GEMV + epilogue */
    SINTER_OP_GDN_STEP = 3,    /* conv+silu, l2norm, gates, delta rule */
    SINTER_OP_ATTN_DECODE = 4, /* qk norm+rope, KV append, split-K, merge, gate */
    SINTER_OP_KIND_COUNT = 5
};

typedef struct sinter_instr {
    uint16_t kind;
    uint16_t block_lo;
    uint16_t block_hi;
    uint16_t flags;
    uint32_t dbg_node;
    uint32_t _pad;
    unsigned char payload[240];
} sinter_instr;

/* SINTER_OP_GEMV prologue modes: how the activation vector a[K] is formed
 * before it is quantised to the weights' vec_dot type (Q8_K for K-quants,
 * Q8_0 for Q8_0, BF16 for BF16, F32 for F32). */
enum sinter_gemv_pro {
    SINTER_PRO_PLAIN = 0,   /* a = x */
    SINTER_PRO_RMSNORM = 1, /* a = rmsnorm(x) * norm_w          (glue.cuh:56-152) */
    SINTER_PRO_GATED = 2,   /* per head of 2^gn_log2d: rmsnorm(x_h)*norm_w*silu(z_h) (gdn.cuh:339-383) */
    SINTER_PRO_EMBED = 3,   /* x = dequant(embd[token]); block_lo writes x_out; a = rmsnorm(x)*norm_w (glue.cuh:202-227) */
    SINTER_PRO_GATED_G = 4  /* as GATED with aux = silu(z) already applied (an EPI_SILU segment made it):
                               per head rmsnorm(x_h)*norm_w*aux_h */
};
/* SINTER_OP_GEMV epilogue modes, per segment */
enum sinter_gemv_epi {
    SINTER_EPI_STORE = 0,  /* y[r] = dot */
    SINTER_EPI_RESID = 1,  /* y[r] = res[r] + dot (residual add fused) */
    SINTER_EPI_SWIGLU = 2, /* y[r] = silu(w.a) * (w2.a)   (gemv.cuh:327-347) */
    SINTER_EPI_ARGMAX = 3, /* y[r] = dot, plus greedy argmax over all rows (harness.cpp:1187-1195) */
    SINTER_EPI_CONV = 4,   /* causal conv + silu per row (channel):          (gdn.cuh:106-171)
                              y[r] = silu(sum_j win_j * w2[r*dconv+j]), win = {aux[r*(dconv-1)..], dot};
                              aux (conv state) <- win[1..] */
    SINTER_EPI_SILU = 5    /* y[r] = silu(dot): the gate of a later GATED_G prologue (gdn.cuh:356-383) */
};

typedef struct sinter_gemv_seg {
    const void *w;   /* weight rows (gate rows for SWIGLU) */
    const void *w2;  /* SWIGLU: up rows; CONV: f32 conv weights [rows][dconv]; else NULL */
    float *y;        /* output rows */
    float *aux;      /* RESID: residual rows (read); CONV: conv state [rows][dconv-1] (updated) */
    uint32_t rows;
    uint8_t type;    /* sinter_type of w (and w2) */
    uint8_t epi;     /* sinter_gemv_epi */
    uint8_t dconv;   /* CONV: taps (2..4) */
    uint8_t _pad;
} sinter_gemv_seg;

#define SINTER_GEMV_MAX_SEG 4
typedef struct sinter_gemv_args {
    const float *x;        /* PLAIN/RMSNORM/GATED input, K floats */
    const float *norm_w;   /* RMSNORM/EMBED: K floats; GATED: 2^gn_log2d floats */
    const void *aux;       /* GATED: z (K floats); EMBED: embedding rows */
    const int32_t *token;  /* EMBED: token id cell */
    float *x_out;          /* EMBED: dequantised row (K floats), written by block_lo */
    void *epi_ws;          /* ARGMAX: sinter_argmax_ws in device memory */
    uint32_t K;
    float eps;
    uint8_t pro;           /* sinter_gemv_pro */
    uint8_t n_seg;
    uint8_t aux_type;      /* EMBED: sinter_type of the embedding rows */
    uint8_t gn_log2d;      /* GATED: log2 of the head width */
    uint32_t aux_rows;     /* EMBED: rows of the embedding (tokens >= aux_rows raise BAD_SHAPE) */
    sinter_gemv_seg seg[SINTER_GEMV_MAX_SEG];
} sinter_gemv_args;

/* Greedy argmax workspace (device memory).  count must be 0 before the first
 * use; the last-arriving block resets it. */
typedef struct sinter_argmax_ws {
    float *part_val;      /* [nblocks] */
    int32_t *part_idx;    /* [nblocks] */
    uint32_t *count;      /* arrival counter */
    int32_t *pass_cell;   /* sinter_pass_cell: token <- argmax, pos += 1, history */
    int32_t *history;     /* tokens produced, indexed by pass_cell->steps */
    uint32_t history_cap;
    uint32_t capacity;    /* partial slots (blocks the workspace was created for) */
    /* forced tokens (prefill): after the pass with pass_cell->steps == s the
     * next token is forced[s + 1] while s + 1 < n_forced, else the argmax;
     * null / 0 for plain greedy decoding */
    const int32_t *forced;
    uint32_t n_forced;
    uint32_t _pad;
} sinter_argmax_ws;

/* Per-pass inputs the kernel reads (harness.cpp:549-566 set_pass_inputs):
 * token and position; the argmax epilogue advances them on device so several
 * greedy passes can run in one launch. */
typedef struct sinter_pass_cell {
    int32_t token;
    int32_t pos;
    int32_t steps;
    int32_t _pad;
} sinter_pass_cell;

/* The causal conv + silu runs in the qkv GEMV epilogue (SINTER_EPI_CONV);
 * this op takes its output. */
typedef struct sinter_gdn_args {
    const float *qkv;       /* [C] conv outputs: q[HK*D] | k[HK*D] | v[HV*D] */
    const float *alpha;     /* [HV] raw ssm_alpha projection */
    const float *beta;      /* [HV] raw ssm_beta projection (pre-sigmoid) */
    const float *dt_bias;   /* [HV] */
    const float *ssm_a;     /* [HV] (= -exp(A_log)) */
    float *state;           /* [HV][D][D] transposed: M[h][col][i] = S[i][col], updated */
    float *o;               /* [HV*D] output, before the gated norm */
    uint32_t hk, hv, d;
    uint32_t cols;          /* columns per work item (divides D; 256 % (D/..) see op) */
    float eps;              /* l2-norm eps */
    float scale;            /* output scale 1/sqrt(D) */
} sinter_gdn_args;

typedef struct sinter_attn_args {
    const float *qg;        /* [NQ][2*HD]: q | gate per head */
    const float *k;         /* [NKV*HD] raw k projection */
    const float *v;         /* [NKV*HD] raw v projection */
    const float *q_norm;    /* [HD] */
    const float *k_norm;    /* [HD] */
    void *kc;               /* K cache [n_ctx][NKV heads]: f16 [HD] or Q8_0 [HD/32 blocks] per head */
    void *vc;               /* V cache, the same layout */
    float *part;            /* partials: [NKV][n_chunks][NQ/NKV][HD+4] fp32 (acc[HD], max, sum, pad);
                               sinter_attn_part_len */
    uint32_t *count;        /* per-(kv head, chunk) generation flags, sinter_attn_count_len words,
                               0 before first use; each call adds 1 to each of the NKV*n_chunks */
    float *out;             /* [NQ*HD] gated attention output */
    const int32_t *pass_cell; /* sinter_pass_cell (pos) */
    uint32_t nq, nkv, hd, rope_dims, n_ctx, n_chunks;
    float theta_scale, eps, scale;
    uint32_t kv_type;       /* SINTER_F16 (also 0) or SINTER_Q8_0 (ggml's f32 -> q8_0 block quantiser on append) */
    uint32_t chunk_min;     /* depth-adaptive split: each chunk spans >= chunk_min positions (whole 32-position
                               tiles), so fewer than n_chunks run at shallow depth; 0 = one tile */
} sinter_attn_args;

/* Buffer sizes for sinter_attn_args (n_chunks <= 64): part in floats,
 * count in 32-bit words.  No counterpart in the reference (its merge reads a
 * fixed 72-way partial array).  The op runs one (kv head, chunk) item per
 * workgroup (blocks >= nkv * n_chunks, all resident: sinter_op_attn_decode
 * launches cooperatively); the chunks of a kv head wait for each other, then
 * each merges a slice of the head group's output. */
size_t   sinter_attn_part_len(uint32_t nq, uint32_t nkv, uint32_t hd, uint32_t n_chunks);
uint32_t sinter_attn_count_len(uint32_t nkv, uint32_t n_chunks);

/* ------------------------------------------------------------------ host control plane */
/* core/host.h:62-80.  Lifecycle: init -> upload -> launch -> run_pass* ->
 * shutdown -> destroy.  On MI355X a pass is one cooperative launch of the
 * interpreter (optionally several greedy passes per launch); launch()
 * validates the program and the cooperative envelope. */
typedef struct sinter_host sinter_host;

int  sinter_host_init(sinter_host **out, int device, unsigned pass_cycles_cap);
int  sinter_host_upload(sinter_host *h, const sinter_instr *prog, uint32_t n_instr,
                        uint32_t epoch_stride);
int  sinter_host_launch(sinter_host *h);
/* returns sinter_run_status */
int  sinter_host_run_pass(sinter_host *h, int32_t token, double timeout_ms);
/* n greedy passes in one launch: tokens_out[i] is the argmax of pass i */
int  sinter_host_run_passes(sinter_host *h, int32_t token, uint32_t n_passes,
                            int32_t *tokens_out, double timeout_ms);
int  sinter_host_shutdown(sinter_host *h, double timeout_ms);
void sinter_host_destroy(sinter_host *h);
int  sinter_host_read_pass_cycles(sinter_host *h, long long *out, unsigned count);
int  sinter_host_reset_op_cycles(sinter_host *h);
/* Diagnostics, no counterpart in the reference (its per-op cycle counters,
 * core/host.h:77-80, are block 0 only): the next launch stamps its first
 * pass into dev_buf (device memory, >= (n_instr+1)*blocks*4 words): for
 * instruction i (i = n_instr: the pass-end barrier) and block b, words
 * [(i*blocks+b)*4 ..] = wall clock (100 MHz) at the instruction's start,
 * after its barrier wait (a barrier fused with the GEMV after it records
 * under the GEMV's index), after a GEMV's prologue (attention: after its q
 * prep; GDN step: after its norms and gates), [2] (attention: after its KV
 * tiles; GDN: after its state update), at its end. */
int  sinter_host_trace_next(sinter_host *h, unsigned long long *dev_buf, size_t words);
int  sinter_host_read_op_cycles(sinter_host *h, long long *out, unsigned count);
/* device pointers the program payloads reference */
sinter_pass_cell *sinter_host_pass_cell(sinter_host *h);
int32_t *sinter_host_history(sinter_host *h, uint32_t *cap);
int  sinter_host_error(sinter_host *h, uint32_t *code, uint32_t *aux);
int  sinter_host_grid(sinter_host *h, uint32_t *blocks, uint32_t *threads, uint32_t *lds_bytes);
/* The interpreter kernel the uploaded program launches (null before an
 * upload): "sinter_interp_kquant" when every GEMV reads Q4_K / Q6_K weights
 * with Q8_K activations and every KV cache is f16, "sinter_interp_kquant_q8kv"
 * for the same over Q8_0 KV caches, "sinter_interp_bf16" for
 * bf16 weights and activations over f16 caches, else the general
 * "sinter_interp".  No counterpart in the reference (one kernel there,
 * core/interp.cu:148-150): the specialised kernels leave out the code of the
 * cases a program does not use. */
const char *sinter_host_kernel(const sinter_host *h);
/* The position of the next run_pass / run_passes: the launch's workgroups
 * write it into the pass cell before their first barrier, as they write the
 * token those calls take (no command of its own on the stream). */
int  sinter_host_set_pos(sinter_host *h, int32_t pos);
/* cooperative grid size (default: one workgroup per CU); before launch() */
int  sinter_host_set_grid(sinter_host *h, uint32_t blocks);
/* Work shares of one GEMV instruction of the uploaded program: block b of its
 * range streams a part of its rows' bytes proportional to share[b] (n = the
 * instruction's block count; each share positive and finite, taken relative to
 * their mean and clamped to [1/16, 16] of it).  Only which workgroup computes
 * which rows changes; every row's value is bit-identical.  Waits for the
 * host's stream.  No counterpart in the reference, whose rows per block are
 * fixed (k0/ops/gemv.cuh:256-321): it is for the static load balance below. */
int  sinter_host_set_gemv_shares(sinter_host *h, uint32_t instr, const float *share, uint32_t n);
/* device time of the last interpreter launch: HIP events recorded on the
 * launch stream immediately before and after the kernel */
float sinter_host_last_launch_ms(sinter_host *h);

/* ------------------------------------------------------------------ op entry points */
/* Each runs one instruction of the given kind over `blocks` workgroups on
 * `stream` (0 = the legacy stream is never used; pass a real hipStream_t).
 * All pointers are device pointers. */
int sinter_op_gemv(const sinter_gemv_args *a, uint32_t blocks, void *stream);
int sinter_op_gdn_step(const sinter_gdn_args *a, uint32_t blocks, void *stream);
int sinter_op_attn_decode(const sinter_attn_args *a, uint32_t blocks, void *stream);
/* Batched GEMV over a ubatch of tokens, the trunk GEMM of a batched prefill
 * (replaces the fork's MMQ prefill GEMM, docs/PREFILL-SEMANTICS.md:286-313:
 * quantised weights times quantised activations on int8 matrix cores).
 * y[t * rows + r] = row r of w (rows x k, SINTER_Q4_K or SINTER_Q6_K, k a
 * multiple of 256) dotted with token t's Q8_K activation (xq + t * (k / 256)
 * blocks of 292 bytes), for t < n_tokens: the single-token GEMV's fp64 item
 * terms folded in item order, so each y[t] is bit-identical to
 * sinter_op_gemv on token t alone.  accumulate != 0: y[t * rows + r] +=
 * the result instead (the RESID epilogue's residual add).  Weights are read
 * once per 64 tokens.
 * Alignment: w 16 bytes (Q4_K) / 4 bytes (Q6_K), xq and y 4 bytes.
 * n_tokens == 0 is a no-op.  SINTER_ERR_ARG on a bad type, shape or
 * alignment (nothing launched). */
int sinter_op_gemv_ubatch(int type, const void *w, int64_t rows, int64_t k, const void *xq,
                          uint32_t n_tokens, float *y, int accumulate, void *stream);
/* The activation side of the same GEMM: x (n_tokens x k f32, row-major,
 * 16-byte aligned, finite) to n_tokens Q8_K activations at xq (k / 256
 * blocks of 292 bytes each, 4-byte aligned), ggml's quantize_row_q8_K_ref
 * (the fork's prefill quantises its activations the same way for MMQ,
 * docs/PREFILL-SEMANTICS.md:303, there to q8_1), bit-identical to the
 * single-token GEMV's Q8_K quantiser.  n_tokens == 0 is a no-op;
 * SINTER_ERR_ARG on a bad shape or alignment. */
int sinter_quant_q8k_ubatch(const float *x, int64_t k, uint32_t n_tokens, void *xq, void *stream);
/* RMSNorm fused ahead of the same quantiser (op_rmsnorm + the activation
 * quantiser, k0/ops/glue.cuh:56-152 and gemv.cuh:213-237, over a ubatch):
 * token t's row x[t] (k f32) is normalised as the single-token GEMV's
 * RMSNORM prologue does (fp32 squares summed in fp64, mean rounded to fp32,
 * scale = 1 / sqrtf(mean + eps), y = (x * scale) * w; w may be NULL for no
 * weight), then quantised to Q8_K at xq.  x and w 16-byte aligned, xq 4. */
int sinter_rmsnorm_quant_q8k_ubatch(const float *x, const float *w, float eps, int64_t k, uint32_t n_tokens,
                                    void *xq, void *stream);
/* SwiGLU fused ahead of the same quantiser (the fused gate/up epilogue,
 * k0/ops/gemv.cuh:327-347, over a ubatch): f = silu(gate) * up elementwise
 * (silu(x) = x / (1 + exp(-x)), the exponential in fp64 as in the
 * single-token GEMV's SWIGLU epilogue), gate and up n_tokens x k f32
 * (16-byte aligned), then quantised to Q8_K at xq for the down projection. */
int sinter_swiglu_quant_q8k_ubatch(const float *gate, const float *up, int64_t k, uint32_t n_tokens, void *xq,
                                   void *stream);
/* The gated RMSNorm of a gated-DeltaNet layer's output (op_gated_rmsnorm,
 * k0/ops/gdn.cuh:356-383, over a ubatch) fused ahead of the same quantiser:
 * per head of head_dim elements (a power of two, 4..256) y = ((x * scale) *
 * w[i]) * silu(z), scale from the head's fp32 squares summed in fp64 (the
 * single-token GEMV's GATED prologue); x and z n_tokens x k f32 (16-byte
 * aligned), w head_dim f32 shared by the heads; Q8_K out at xq. */
int sinter_gated_rmsnorm_quant_q8k_ubatch(const float *x, const float *z, const float *w, uint32_t head_dim,
                                          float eps, int64_t k, uint32_t n_tokens, void *xq, void *stream);
/* The causal conv + silu of a gated-DeltaNet layer's qkv channels over a
 * ubatch (k0/ops/gdn.cuh:106-171, token after token): x and y n_tokens x
 * channels f32; state channels x (dconv - 1) f32, read and left holding the
 * last dconv - 1 inputs; conv_w channels x dconv f32 (tap-contiguous);
 * dconv 1..8.  Token t's row equals the single-token GEMV's CONV epilogue
 * after tokens 0..t-1. */
int sinter_conv_silu_ubatch(const float *x, float *state, const float *conv_w, float *y, int64_t channels,
                            uint32_t dconv, uint32_t n_tokens, void *stream);
/* The attention op without caller workspace, allocating nothing: no
 * counterpart in the reference; for callers that cannot allocate device
 * memory (tight serving loops, harnesses that forbid allocation; it launches
 * cooperatively and takes the array's address on its first call per device,
 * so it is not offered for HIP graph capture).  As sinter_op_attn_decode,
 * except that a->part and
 * a->count must be NULL: the split-K partials (at most 2 MiB,
 * sinter_attn_part_len(...) * 4 bytes) and the generation flags (at most
 * 1024, sinter_attn_count_len(...)) live in a fixed device array the library
 * holds on each GPU it runs on until the process ends; larger shapes are
 * refused with SINTER_ERR_ARG.  Every call on a GPU shares that array (its
 * flags are cleared by a small kernel at the start of each call): calls that
 * overlap on one GPU race.  Errors go to the cell sinter_op_error reads. */
int sinter_op_attn_decode_noalloc(const sinter_attn_args *a, uint32_t blocks, void *stream);
/* Counter calibration (a diagnostic, no counterpart in the reference): on
 * `device`, copies `bytes` device-to-device `reps` times with the runtime's
 * copy kernel, so that FETCH_SIZE / WRITE_SIZE of a copy of known size can
 * scale the same counters read on the interpreter. */
int sinter_copy_calibration(int device, size_t bytes, int reps);

/* Measured HBM bandwidth on the current device (a diagnostic, no counterpart
 * in the reference, which quotes its practical peak from a copy benchmark,
 * k0/ops/NOTES-gemv.md:58-72): `bytes` (>= 64 MiB, rounded down to 16 MiB)
 * of device memory read by a streaming kernel `reps` times, and copied half
 * to half `reps` times, after one untimed pass of each.  read_gbs = bytes
 * read / time; copy_gbs = bytes read + written / time (1e9 B/s).  Buffers
 * well past the 256 MB memory-side cache measure HBM. */
int sinter_hbm_peak(uint64_t bytes, uint32_t reps, double *read_gbs, double *copy_gbs);
/* Grid-barrier litmus on the current device (mirrors tests/litmus_boundary.cu:1-18
 * and docs/SYNC-FINDINGS.md:9-32 of the reference; a diagnostic, not a decode
 * entry point).  `blocks` co-resident workgroups cross the interpreter's grid
 * barrier `epochs` times with pseudo-random arrival order; each publishes a
 * payload word before arriving and, after crossing, reads the next block's
 * (another XCD's).  `mode` is one of the SINTER_LITMUS_* protocols, or'ed with
 * the kind of read the reader makes of that line before arriving (none, plain
 * cached, or coherent): it leaves the previous epoch's value wherever that read
 * caches it.  counts[0] = payload reads older than the current epoch (stale),
 * counts[1] = crossings that saw fewer than epoch*blocks arrivals counted
 * (early release), counts[2] = the final arrival count (epochs*blocks).
 * COHERENT is the protocol the ops use (both counts must be 0); the other
 * protocols break only the payload's visibility. */
enum {
    SINTER_LITMUS_COHERENT = 0,       /* sc1 store before arriving, sc1 load after crossing */
    SINTER_LITMUS_PLAIN_STORE = 1,    /* plain cached store */
    SINTER_LITMUS_PLAIN_LOAD = 2,     /* plain cached load */
    SINTER_LITMUS_LATE_PUBLISH = 3,   /* store after arriving */
    SINTER_LITMUS_WARM_PLAIN = 0x10,  /* pre-read: plain cached load */
    SINTER_LITMUS_WARM_COHERENT = 0x20 /* pre-read: sc1 load */
};
int sinter_litmus_barrier(uint32_t blocks, uint32_t epochs, int mode, uint64_t counts[3]);
/* synchronise the device and read/clear the op error cells of the current device */
int sinter_op_error(uint32_t *code, uint32_t *aux);
/* argmax workspace for `blocks` workgroups (allocated on the current device) */
int sinter_argmax_ws_create(uint32_t blocks, int32_t *pass_cell, int32_t *history,
                            uint32_t history_cap, sinter_argmax_ws **out_dev);
void sinter_argmax_ws_destroy(sinter_argmax_ws *dev);

/* ------------------------------------------------------------------ synthetic data */
/* Deterministic synthetic tensors (integer hashing plus exactly rounded fp32
 * arithmetic, so host and device produce identical bytes).  kind selects the
 * distribution; see sinter_synth_kind. */
enum sinter_synth_kind {
    SINTER_SYN_WEIGHT = 0,  /* quantised weight rows of `type`, ~N(0, 0.02) scale */
    SINTER_SYN_Q8_0_CFG1 = 1,/* Q8_0: codes U[-127,127], d = f16(|N(0, 0.02)|) */
    SINTER_SYN_NORMAL = 2,  /* f32 ~ mean + std * N(0,1) (Irwin-Hall(4) approximation) */
    SINTER_SYN_UNIFORM = 3, /* f32 ~ U[lo, hi) */
    SINTER_SYN_NORMAL_F16 = 4,/* f16 ~ std * N(0,1) */
    SINTER_SYN_NORMAL_Q8_0 = 5 /* Q8_0 blocks of std * N(0,1) (ggml's q8_0 quantiser); k a multiple of 32 */
};
/* Fill n elements (rows*k for weights) at dst.  dev != 0: dst is device
 * memory and the fill runs on `stream`; dev == 0: host memory. */
int sinter_synth(int dev, void *dst, int kind, int type, int64_t rows, int64_t k,
                 uint64_t seed, float a, float b, void *stream);
uint64_t sinter_seed(uint64_t config_id, const char *tensor_name, int64_t layer);

/* ------------------------------------------------------------------ model */
/* default of sinter_model_config.attn_chunk_min: the split-K attention gives
 * each chunk at least this many KV positions */
#define SINTER_ATTN_CHUNK_MIN 128

typedef struct sinter_model_config {
    int32_t n_layer, attn_every, n_embd, n_ff, n_vocab;
    int32_t gdn_hk, gdn_hv, gdn_d, conv_k;
    int32_t attn_nq, attn_nkv, head_dim, rope_dims;
    float rope_base, eps;
    int32_t n_ctx;
    int32_t t_default, t_attn_v, t_ffn_down, t_output, t_embd;
    int32_t t_kv;           /* KV cache type: SINTER_F16 (also when 0) or SINTER_Q8_0 */
    int32_t attn_chunks;    /* split-K chunks per kv head at most (1..64; 0: min(64, workgroups / attn_nkv)) */
    int32_t attn_chunk_min; /* positions per chunk at least (depth-adaptive split; 0: SINTER_ATTN_CHUNK_MIN) */
} sinter_model_config;

typedef struct sinter_model sinter_model;

/* Allocates weights (synthesised on device from seed), state and buffers,
 * compiles and uploads the pass program. */
int  sinter_model_create(const sinter_model_config *cfg, int device, uint64_t seed,
                         uint32_t blocks, sinter_model **out);
void sinter_model_destroy(sinter_model *m);
/* one pass: writes logits (host, n_vocab floats, nullable) and the greedy id */
int  sinter_model_decode(sinter_model *m, int32_t token, int32_t pos, float *logits_host,
                         int32_t *next_token);
/* n greedy passes from (token, pos) in one launch */
int  sinter_model_greedy(sinter_model *m, int32_t token, int32_t pos, uint32_t n,
                         int32_t *tokens_out);
/* A model over caller-owned device memory (the drop-in path: a host
 * framework's weight, KV-cache and recurrent-state tensors, by raw pointer;
 * k0/harness.cpp:589-628 resolves program names to pointers the same way).
 * The model allocates only its activations, scratch and control cells and
 * never frees or fills the bound buffers. */
typedef struct sinter_model_bindings {
    void *const *tensors;    /* [n_layer * 16 + 3] device pointers, numbered as sinter_model_tensor_info
                                (16-byte aligned; null for slots the layer kind lacks, and for the
                                embedding when embed_outside) */
    const int32_t *types;    /* the same count: each weight's sinter_type (vectors SINTER_F32) */
    void *const *states;     /* [n_layer * 2]: conv / recurrent state (GDN layers), K / V cache
                                (attention layers) in the sizes sinter_model_state_info reports */
    float *logits;           /* n_vocab floats the head writes (null: the model allocates them) */
    uint32_t embed_outside;  /* 1: the pass starts from the embedded row (n_embd floats) the caller
                                writes into the "X" buffer (sinter_model_buffer) before it */
    uint32_t _pad;
} sinter_model_bindings;
int  sinter_model_create_bound(const sinter_model_config *cfg, int device, uint32_t blocks,
                               const sinter_model_bindings *b, sinter_model **out);
/* Prefill on the GPU: tokens[0..n) at positions pos0.., the greedy
 * continuation of the last one in *next_token (may be null), its logits in
 * the model's logits buffer (sinter_model_logits).  The KV rows, the
 * recurrent and conv states and the logits are bit-identical to decoding the
 * tokens one by one.  Batched (sinter_model_prefill_batched with
 * SINTER_PREFILL_UBATCH tokens per ubatch) when every matrix of the model is
 * Q4_K or Q6_K, else the decode passes (sinter_model_prefill_tokenwise).
 * Replaces the prompt stage of the reference's server
 * (docs/PREFILL-SEMANTICS.md:23-57, 379-426). */
int  sinter_model_prefill(sinter_model *m, const int32_t *tokens, uint32_t n, int32_t pos0,
                          int32_t *next_token);
/* The decode program over the prompt: one pass per token with each pass's
 * next token forced to the prompt's (the reference's "(b)" token loop for
 * every layer); launches run up to the history capacity's passes each. */
int  sinter_model_prefill_tokenwise(sinter_model *m, const int32_t *tokens, uint32_t n, int32_t pos0,
                                    int32_t *next_token);
/* The batched prefill: ubatches of up to `ubatch` tokens (1..SINTER_PREFILL_UBATCH_MAX),
 * each layer once per ubatch -- RMSNorm + Q8_K, the trunk GEMMs on int8 MFMA
 * (sinter_op_gemv_ubatch), the conv and the gated-DeltaNet recurrence token
 * after token in one launch per layer, q/k norm + RoPE + the KV append, and
 * causal attention split per query as the decode splits it -- then the head
 * on the last token.  SINTER_ERR_ARG for a model with a matrix of another
 * type (Q8_0, BF16, F32) or embedded outside. */
#define SINTER_PREFILL_UBATCH 256
#define SINTER_PREFILL_UBATCH_MAX 1024
int  sinter_model_prefill_batched(sinter_model *m, const int32_t *tokens, uint32_t n, int32_t pos0,
                                  uint32_t ubatch, int32_t *next_token);
/* the logits of the last pass (n_vocab floats to host): the result_output
 * cell of k0/program.json, read after run_pass / greedy */
int  sinter_model_logits(sinter_model *m, float *logits_host);
/* fill KV caches / recurrent states with seeded synthetic values, as if a
 * context of n_past tokens had been prefilled */
int  sinter_model_synth_context(sinter_model *m, int32_t n_past, uint64_t seed);
/* host access to the tensors the oracle needs (slot numbering as
 * oracle/oracle.h: layer*16 + slot; globals at n_layer*16 + {0,1,2}) */
int  sinter_model_tensor_info(sinter_model *m, int64_t layer, int slot, void **dev_ptr,
                              size_t *bytes, int *type);
int  sinter_model_state_info(sinter_model *m, int64_t layer, int slot, void **dev_ptr,
                             size_t *bytes);
int  sinter_model_copy(sinter_model *m, void *dst, const void *src, size_t bytes, int dir);
int  sinter_model_info(sinter_model *m, uint64_t *weight_bytes, uint32_t *n_instr,
                       uint32_t *n_boundaries, uint32_t *blocks);
sinter_host *sinter_model_host(sinter_model *m);
/* Static load balance of the model's GEMVs: rounds + 1 measurements of
 * `traces` traced greedy passes each from (*token, *pos) (both advanced by
 * (rounds + 1) * traces); after each of the first `rounds` every workgroup's
 * GEMV share is rescaled so that the workgroups would end together
 * (sinter_host_set_gemv_shares), and a GEMV shape whose tail got longer keeps
 * its best shares.  Results are unchanged. */
int sinter_model_balance(sinter_model *m, int32_t *token, int32_t *pos, uint32_t rounds, uint32_t traces);
/* the configuration the model was created with */
int sinter_model_get_config(sinter_model *m, sinter_model_config *cfg);
/* The symbolic-program packer's view of a model (k0/harness.cpp:589-628 resolves
 * the reference's buf:/cell: names the same way): the device buffer behind an
 * activation / workspace name -- X, H (residual stream), qkv, z, alpha, beta,
 * o (GDN), qg, k, v, att (attention), ffn, logits, attn_part, attn_count,
 * argmax_ws -- and a copy of the model's uploaded program (n_instr always
 * set; out may be null). */
int sinter_model_buffer(sinter_model *m, const char *name, void **dev_ptr, size_t *bytes);
int sinter_model_program(sinter_model *m, sinter_instr *out, uint32_t cap, uint32_t *n_instr);
/* Single-op benchmark programs for BASELINE configs 1-3 (no counterpart in the
 * reference, whose op timings come from its own harness): replaces the
 * model's program (its decode program is gone afterwards) with, for every
 * layer, one op group between grid barriers, so consecutive groups read
 * different weight copies (rotate >= 4 copies past the 256 MB MALL):
 *   GEMV  y = W x over the layer's ffn_gate matrix (n_ff x n_embd, plain
 *         prologue, stored output; config 1 with t_default = Q8_0),
 *   GDN   the gated-DeltaNet mixer of every GDN layer: norm + projections,
 *         the recurrent step, gated norm + output projection (config 2),
 *   ATTN  the attention mixer of every attention layer (config 3).
 * x ~ N(0,1) from `seed`; states and caches as sinter_model_synth_context
 * left them.  Time it with sinter_host_set_pos + sinter_host_run_passes on
 * sinter_model_host(m) and sinter_host_last_launch_ms. */
enum { SINTER_BENCH_GEMV = 1, SINTER_BENCH_GDN = 2, SINTER_BENCH_ATTN = 3 };
int sinter_model_bench_program(sinter_model *m, int kind, uint64_t seed);

/* ------------------------------------------------------------------ GGUF */
/* A read-only GGUF v3 file (k0/gguf.h:30-246 File::open/parse/find/find_kv,
 * with the K-quant, Q8_0 and BF16 block sizes added).  The file is
 * memory-mapped; tensor data pointers point into the mapping and stay valid
 * until sinter_gguf_close.  Malformed files (magic, version, truncation,
 * unknown tensor type, partial blocks, misaligned or out-of-file data) are
 * refused with SINTER_ERR_ARG. */
typedef struct sinter_gguf sinter_gguf;
typedef struct sinter_gguf_tensor {
    const char *name;     /* owned by the handle */
    uint32_t type;        /* ggml type id (sinter_type numbering) */
    uint32_t n_dims;
    uint64_t ne[4];       /* ne[0] = elements per row */
    uint64_t offset;      /* from the start of the data section */
    uint64_t nbytes;
    const void *data;     /* host pointer into the mapping */
} sinter_gguf_tensor;
int  sinter_gguf_open(const char *path, sinter_gguf **out);
void sinter_gguf_close(sinter_gguf *g);
int  sinter_gguf_info(sinter_gguf *g, uint32_t *version, uint64_t *n_tensors, uint64_t *n_kv, uint64_t *alignment);
int  sinter_gguf_get_tensor(sinter_gguf *g, uint64_t i, sinter_gguf_tensor *out);
/* index of the named tensor, or -1 */
int64_t sinter_gguf_find(sinter_gguf *g, const char *name);
int  sinter_gguf_kv_i64(sinter_gguf *g, const char *key, int64_t *out);   /* integer or bool */
int  sinter_gguf_kv_f64(sinter_gguf *g, const char *key, double *out);    /* any number */
int  sinter_gguf_kv_str(sinter_gguf *g, const char *key, char *buf, size_t n);
/* integer array: copies min(cap, length) values, *n = length */
int  sinter_gguf_kv_arr_i64(sinter_gguf *g, const char *key, int64_t *out, size_t cap, size_t *n);
/* The model shape of a GGUF file (k0/harness.cpp:315-400 Residency): sizes
 * from the tensor table -- n_embd and n_vocab from token_embd, blocks from
 * blk.N.attn_norm (less <arch>.nextn_predict_layers), attention blocks from
 * blk.N.attn_q (every attn_every-th), head sizes from the q/k norms, the
 * gated-DeltaNet heads from ssm_norm / ssm_a / attn_qkv -- and rope
 * dimensions, rope base and the RMS eps from <arch>.rope.dimension_count,
 * <arch>.rope.freq_base, <arch>.attention.layer_norm_rms_epsilon. */
int  sinter_model_config_from_gguf(sinter_gguf *g, int32_t n_ctx, sinter_model_config *cfg);
/* A model whose weights are the file's tensors, uploaded as they lie in the
 * file (GGUF names blk.N.<name>.weight, ssm_dt.bias, ssm_a; without
 * output.weight the head is token_embd).  Each tensor keeps its own type
 * (Q4_K, Q6_K, Q8_0, BF16 or F32 weights; F32 norms and conv weights); the
 * segments of one fused GEMV must share an activation type.  The file may be
 * closed after this returns. */
int  sinter_model_create_from_gguf(sinter_gguf *g, int device, int32_t n_ctx, uint32_t blocks, sinter_model **out);

#ifdef __cplusplus
}
#endif
#endif
