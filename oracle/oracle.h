/*
 * CPU ORACLE -- test infrastructure only.
 *
 * A plain-C restatement of the ggml CPU semantics that the reference's decode
 * pass computes (ggml is not vendored in the reference; see the per-function
 * citations in oracle.c).  It is the checker for the HIP path: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and the
 * product never routes through it.
 *
 * Declared numerics (shared with the HIP kernels, restated independently):
 *   - quantised dot products: exact integer block sums; one fp64 term per
 *     block c_b = (d_w * d_x) * isum [- (dmin * d_x) * imin], blocks summed
 *     in ascending order in fp64, rounded to fp32 once per output row;
 *   - every other sum of products is accumulated in fp64 from exact products
 *     and rounded to fp32 once;
 *   - exp/log/sin/cos are evaluated in fp64 (libm here, ocml on the GPU) and
 *     rounded to fp32 where the ggml op works in fp32.
 * With these rules the result does not depend on summation order except at
 * the fp64 rounding level, so GPU and CPU agree bit-for-bit except with a
 * probability of order 1e-8 per output.
 */
#ifndef SINTER_ORACLE_H
#define SINTER_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* weight/activation type ids (same numbering as include/sinter.h) */
enum { OR_F32 = 0, OR_F16 = 1, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q6_K = 14, OR_Q8_K = 15, OR_BF16 = 30 };

/* scalar conversions */
float    or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
float    or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);
int      or_nearest_int(float f);

/* block geometry */
size_t or_type_block_elems(int type);
size_t or_type_block_bytes(int type);
size_t or_row_bytes(int type, int64_t k);

/* dequantisation of one row of k elements */
void or_dequant_row(int type, const void *row, float *out, int64_t k);

/* activation quantisers */
void or_quant_q8_0(const float *x, void *y, int64_t k);  /* x86 AVX2 form */
void or_quant_q8_0_ref(const float *x, void *y, int64_t k);  /* reference form (KV cache rows) */
void or_quant_q8_K(const float *x, void *y, int64_t k);  /* reference form */
void or_quant_bf16(const float *x, uint16_t *y, int64_t k);

/* one block's fp64 dot term (declared fold) */
double or_block_term(int type, const void *wblk, const void *xblk);

/* y[r] = W[r,:] . x for r in [0, rows); x is quantised inside to the type's
 * vec_dot type.  Multi-threaded over rows (results are thread-count free). */
void or_gemv(int type, const void *w, int64_t rows, int64_t k, const float *x, float *y);
/* the ISA of the GEMV row kernels on this CPU: 512 (AVX-512) or 0 (baseline) */
int or_row_isa(void);
/* same, over an already quantised activation */
void or_gemv_q(int type, const void *w, int64_t rows, int64_t k, const void *xq, float *y);

/* normalisations and unary ops */
void  or_rmsnorm(const float *x, const float *w, float *y, int64_t n, float eps);
void  or_l2norm(const float *x, float *y, int64_t n, float eps);
float or_silu(float x);
float or_sigmoid(float x);
float or_softplus(float x);

/* gated-DeltaNet pieces */
void or_conv_silu(const float *xnew, float *conv_state, const float *conv_w,
                  float *out, int64_t channels, int dconv);
void or_gdn_gates(const float *alpha, const float *beta_raw, const float *dt_bias,
                  const float *ssm_a, float *g, float *beta, int nh);
/* state M[h][col][i] = S[i][col], updated in place; o[h*dv + col]; the fp32
 * folds follow the kernel's layout of cols columns per 256-thread item */
void or_gdn_step(const float *q, const float *k, const float *v, const float *g,
                 const float *beta, float *state, float *o, int hv, int hk, int d,
                 float scale, int cols);
int or_gdn_cols(int d);
void or_gated_rmsnorm(const float *x, const float *z, const float *w, float *y,
                      int nh, int d, float eps);

/* attention pieces */
float or_rope_theta_scale(float freq_base, int n_dims);
void  or_rope_neox(float *x, int hd, int n_dims, int pos, float theta_scale);
void  or_attn_decode(const float *q, const uint16_t *kc, const uint16_t *vc,
                     int n_kv, int nq, int nkv, int hd, int row_width, float scale,
                     float *out);
/* the same over a cache of kv_type OR_F16 or OR_Q8_0 (rows of nkv*hd
 * elements; a Q8_0 element is dequantised exactly first) */
void  or_attn_decode_kv(const float *q, const void *kc, const void *vc, int kv_type,
                        int n_kv, int nq, int nkv, int hd, float scale, float *out);

/* the fp32 split-K attention of the GPU op (declared folds, see oracle.c):
 * out[nq][hd] = the un-gated attention over n_kv positions in at most
 * n_chunks chunks of >= chunk_min positions; or_attn_geom gives the tiles,
 * tiles per chunk and chunk count */
void  or_attn_geom(int n_kv, int n_chunks, int chunk_min, int *tiles, int *tpc, int *nch);
void  or_attn_split(const float *q, const void *kc, const void *vc, int kv_type, int n_kv, int nq,
                    int nkv, int hd, float scale, int n_chunks, int chunk_min, float *out);

/* model configuration (mirrors sinter_model_config in include/sinter.h) */
typedef struct {
    int32_t n_layer, attn_every, n_embd, n_ff, n_vocab;
    int32_t gdn_hk, gdn_hv, gdn_d, conv_k;
    int32_t attn_nq, attn_nkv, head_dim, rope_dims;
    float   rope_base, eps;
    int32_t n_ctx;
    int32_t t_default, t_attn_v, t_ffn_down, t_output, t_embd;
    int32_t t_kv;   /* KV cache: OR_F16 (also 0) or OR_Q8_0 */
    int32_t attn_chunks, attn_chunk_min;   /* split-K attention geometry (or_attn_split) */
} or_cfg;

/* per-layer weight slots (NSLOT pointers per layer) */
enum {
    OR_SLOT_ATTN_NORM = 0, OR_SLOT_POST_NORM, OR_SLOT_FFN_GATE, OR_SLOT_FFN_UP,
    OR_SLOT_FFN_DOWN,
    /* gated-DeltaNet layers */
    OR_SLOT_QKV = 5, OR_SLOT_Z, OR_SLOT_ALPHA, OR_SLOT_BETA, OR_SLOT_SSM_OUT,
    OR_SLOT_CONV_W, OR_SLOT_DT_BIAS, OR_SLOT_SSM_A, OR_SLOT_SSM_NORM,
    /* attention layers */
    OR_SLOT_WQ = 5, OR_SLOT_WK, OR_SLOT_WV, OR_SLOT_WO, OR_SLOT_Q_NORM, OR_SLOT_K_NORM,
    OR_NSLOT = 16
};
/* per-layer state slots: GDN {conv f32[C*(dconv-1)], ssm f32[hv*d*d]};
 * attention {K f16[n_ctx*nkv*hd], V f16[n_ctx*nkv*hd]} */
enum { OR_ST_CONV = 0, OR_ST_SSM = 1, OR_ST_K = 0, OR_ST_V = 1, OR_NST = 2 };

int or_is_attn_layer(const or_cfg *c, int il);

/* one sublayer (mixer) on a normalised input; writes the mixer output */
void or_gdn_mixer(const or_cfg *c, const void *const *w, void *const *st,
                  const float *xn, float *out, float *dbg /* nullable, see .c */);
void or_attn_mixer(const or_cfg *c, const void *const *w, void *const *st,
                   const float *xn, int pos, float *out, float *dbg);
void or_ffn(const or_cfg *c, const void *const *w, const float *xn, float *out);

/* full decode pass: embedding -> layers -> norm -> head -> argmax.
 * weights: n_layer*OR_NSLOT slots then {embd, out_norm, output};
 * state:   n_layer*OR_NST slots.  resid (nullable): n_layer*n_embd layer outputs. */
int or_decode_step(const or_cfg *c, const void *const *weights, void *const *state,
                   int token, int pos, float *logits, float *resid);

int64_t or_argmax_first(const float *x, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
