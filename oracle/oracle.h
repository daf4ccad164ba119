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

/* ---- thread pool used by both models ---- */
void orc_set_threads(int n);
int  orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
