/* oracle.h — CPU restatement of redukt's Mamba-1 and RWKV-7 CPU step.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity oracle and the timed CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it; the product library (libredukt_gpu.so) never links or calls it.
 *
 * Every function follows the operation order of the reference CPU path; the file
 * and line each one restates are cited at the definition in mamba_oracle.c and
 * rwkv7_oracle.c.
 */
#ifndef REDUKT_ORACLE_H
#define REDUKT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight profiles (bit field).  Low two bits: 0 = F32, 1 = Q8 with one scale per
 * 64 columns (the reference's Q8 profile), 2 = Q8 with one scale per output row.
 * Bit 2: also quantize x_proj and dt_proj (the reference keeps them f32). */
enum {
    ORC_PROFILE_F32 = 0,
    ORC_PROFILE_Q8_G64 = 1,
    ORC_PROFILE_Q8_ROW = 2,
    ORC_PROFILE_Q8_SMALL = 4,
    /* RWKV-7 with per-row int8 weights only: int8 activations as well (W8A8,
     * tensor.rs:1791-1866), the reference's own RWKV-7 Q8 arithmetic. */
    ORC_PROFILE_W8A8 = 32,
    /* Mamba: the reference-order tier of the GPU library.  The oracle always computes in
     * the reference order, so this bit changes nothing here; it is accepted so that the
     * oracle and the library take the same profile words. */
    ORC_PROFILE_EXACT = 64,
    /* Mamba: every GEMV in numeric contract 2 (fma-v1, gemv_fma.rs) instead of 1. */
    ORC_PROFILE_FMA = 128,
};

/* ---- scalar math (tensor.rs) ---- */
float orc_expf(float x);
float orc_lnf(float x);
float orc_lane_expf(float x);
float orc_sigmoidf(float x);
float orc_softplus(float x);
void  orc_softmax_into(const float* logits, float* out, int n);

/* ---- kernels (gemv.rs / tensor.rs) ---- */
float orc_dot_f32(const float* w, const float* v, int n);
/* q: rows*cols int8, scales: rows*(cols/group) */
void  orc_quantize(const float* w, int rows, int cols, int group, int8_t* q, float* scales, int* group_out);
void  orc_gemv_f32(const float* w, int rows, int cols, const float* v, float* out);
void  orc_gemv_q8(const int8_t* q, const float* scales, int rows, int cols, int group,
                  const float* v, float* out);
/* The same GEMVs in numeric contract 2 (fma-v1, gemv_fma.rs:98-134). */
float orc_dot_f32_fma(const float* w, const float* v, int n);
void  orc_gemv_f32_fma(const float* w, int rows, int cols, const float* v, float* out);
void  orc_gemv_q8_fma(const int8_t* q, const float* scales, int rows, int cols, int group,
                      const float* v, float* out);
void  orc_rms_norm(float* x, const float* w, int n, float eps);
void  orc_layer_norm(float* out, const float* x, const float* w, const float* b, int n, float eps);
void  orc_ssm_d16(float* y, float* ss, const float* dt, const float* conv_out, const float* a_log,
                  const float* b, const float* c, const float* d_vec, int d_inner);

/* ---- Mamba model (mamba/model.rs) ---- */
typedef struct OrcMamba OrcMamba;
/* err: 0 ok, 4 weights not found / bad header, 1 out of memory */
OrcMamba* orc_mamba_load(const char* rbin_path, int profile, int* err);
void      orc_mamba_free(OrcMamba* m);
/* vocab, d_model, d_inner, d_state, d_conv, dt_rank, n_layer, flags */
void      orc_mamba_dims(const OrcMamba* m, uint32_t out[8]);
int       orc_mamba_pool_init(OrcMamba* m, uint32_t cap);
/* Zero the listed slots (NULL = all). */
int       orc_mamba_reset(OrcMamba* m, const uint32_t* slots, uint32_t n);
/* Periodic reset period in forwards per slot (0 = never), mamba/model.rs:315-320. */
void      orc_mamba_set_reset_every(OrcMamba* m, uint64_t every);
/* One lockstep step; out = n*vocab logits, row b = stream b.  Returns 0 or 5. */
int       orc_mamba_forward(OrcMamba* m, uint32_t n, const uint32_t* slots, const uint32_t* tokens,
                            float* out_logits);
/* Copy a slot's state of one layer: conv (d_inner*(d_conv-1)), ssm (d_inner*d_state). */
int       orc_mamba_get_state(const OrcMamba* m, uint32_t slot, uint32_t layer, float* conv, float* ssm);
/* Dequantized view of the quantized weights (for tests): which = 0 in_proj, 1 out_proj,
 * 2 emb, 3 x_proj, 4 dt_proj; layer ignored for emb.  Writes rows*cols floats. */
int       orc_mamba_dequant(const OrcMamba* m, int which, uint32_t layer, float* out);

/* ---- RWKV-7 element-wise helpers (tensor.rs; 8-aligned body in lane form) ---- */
void  orc_tanh_inplace(float* x, int n);
void  orc_sigmoid_inplace(float* x, int n);
void  orc_sigmoid_add_into(float* out, const float* base, const float* offset, int n);
void  orc_decay_sigmoid_into(float* out, const float* base, const float* offset, int n);
void  orc_sigmoid_mix_inplace(float* v, const float* v_first, const float* base, const float* offset, int n);
void  orc_group_norm_into(float* out, const float* x, int groups, const float* w, const float* b, int n, float eps);
void  orc_l2_normalize_per_head(float* x, int heads, int hs);
void  orc_mat_vec_small(float* out, const float* a, const float* v, int n);
/* One head's WKV-7 update and read-out; tmp holds 3n floats. */
void  orc_wkv_head(float* S, int n, const float* r, const float* w, const float* kk, const float* a,
                   const float* v, const float* kmod, float* out, float* tmp);
float orc_lane_sigmoidf(float x);
/* W8A8 (tensor.rs:1791-1866): quantize v[0..n) to q with one scale (returned); then
 * out[r] = (float)(exact int32 q[r]·vq) * (scales[r] * v_scale) for a per-row int8 matrix. */
float orc_quantize_vec_i8(const float* v, int n, int8_t* q);
void  orc_q8_matvec_a8(const int8_t* q, const float* scales, int rows, int cols, const int8_t* vq, float v_scale,
                       float* out);

/* ---- RWKV-7 model (rwkv7/model.rs) ---- */
typedef struct OrcRwkv OrcRwkv;
/* NULL on a missing file, a bad header or a short/long body. */
OrcRwkv*  orc_rwkv_load(const char* path, int profile);
void      orc_rwkv_free(OrcRwkv* m);
/* vocab, d_model, n_head, head_size, n_layer, d_ffn, lora w/a/v/g ranks, g1k */
void      orc_rwkv_dims(const OrcRwkv* m, uint32_t out[11]);
int       orc_rwkv_pool_init(OrcRwkv* m, uint32_t cap);
int       orc_rwkv_reset(OrcRwkv* m, const uint32_t* slots, uint32_t n);
void      orc_rwkv_set_reset_every(OrcRwkv* m, uint64_t every);
int       orc_rwkv_forward(OrcRwkv* m, uint32_t n, const uint32_t* slots, const uint32_t* tokens,
                           float* out_logits);
/* A slot's state of one layer: token-shift inputs of the two mixers (d_model each) and
 * the WKV matrices [n_head][head_size][head_size] (row i, column j as the reference). */
int       orc_rwkv_get_state(const OrcRwkv* m, uint32_t slot, uint32_t layer, float* x_att, float* wkv,
                             float* x_ffn);

/* ---- thread pool used by both models ---- */
void orc_set_threads(int n);
int  orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
