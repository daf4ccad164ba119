/* rwkv7_oracle.c — CPU restatement of redukt's RWKV-7 single-token step.
 *
 * TEST INFRASTRUCTURE ONLY (parity oracle and CPU baseline of libredukt_gpu.so).
 *
 * Follows src/infrastructure/rwkv7/model.rs:643-925 (forward_into, time_mixing_scratch,
 * channel_mixing_scratch) operation for operation, with the element-wise helpers of
 * src/domain/tensor.rs (cited at each use) and the GEMV orders of the Mamba part:
 * f32 matrices in dot_avx2_order (tensor.rs:1680-1693, used by mat_vec_mul_into at
 * :1602-1705), int8 weight-only matrices in the q8w order (gemv.rs:490-502).  The reference
 * quantizes RWKV-7 as W8A8 (tensor.rs:105-143, 1791-1866): with profile bit 5 the per-row
 * int8 matrices take that path (each input vector quantized to int8 with one scale, exact
 * int32 dot products, one f32 rescale per row).  Without it the int8 profiles are the
 * weight-only recipe of the Mamba path.  Either way the quantized matrices are the ones the
 * reference quantizes (receptance, key, value, output, FFN key/value, head; LoRAs and the
 * embedding stay f32, model.rs:1004-1058).
 *
 * Weight file: the RWKV-7 container of redukt_amd/rwkv.py (64-byte header, then f32
 * tensors in that module's tensor_order).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "internal.h"
#include "oracle.h"
#include "pool.h"

#define RWKV_MAGIC 0x55504752u
#define RWKV_VERSION 3u
#define RWKV_MODEL 2u

typedef struct {
    float *ln1_w, *ln1_b, *ln2_w, *ln2_b;
    float *x_r, *x_w, *x_k, *x_v, *x_a, *x_g;
    float *w0, *w1, *w2, *a0, *a1, *a2, *v0, *v1, *v2, *g1, *g2;
    float *k_k, *k_a, *r_k;
    Mat r, k, v, o;
    float *ln_x_w, *ln_x_b, *ffn_x_k;
    Mat fk, fv;
} RLayer;

struct OrcRwkv {
    uint32_t vocab, d, h, n, nl, f, rw, ra, rv, rg, g1k;
    int profile;
    float* emb;         /* [V][D], already through ln0 */
    RLayer* layers;
    float *ln_out_w, *ln_out_b;
    Mat head;
    uint32_t cap;
    float* x_att;       /* [slot][layer][D] */
    float* wkv;         /* [slot][layer][H][N][N] */
    float* x_ffn;       /* [slot][layer][D] */
    float* v_first;     /* [slot][D] */
    uint64_t* since;
    uint64_t reset_every;
};

/* ---- element-wise helpers (tensor.rs), exported for the tests ---- */

/* Elements the reference's AVX2 kernels take in 8-wide lanes (simd_body_len, :895-898);
 * lane functions there, portable ones on the tail. */
static inline int body_len(int n) { return n / 8 * 8; }

static inline float portable_sigmoidf(float x) { return 1.0f / (1.0f + orc_expf(-x)); }  /* :842-845 */
static inline float portable_tanhf(float x) { return 2.0f * portable_sigmoidf(2.0f * x) - 1.0f; } /* :847-850 */
static inline float lane_tanhf(float x) { return orc_lane_sigmoidf(x * 2.0f) * 2.0f - 1.0f; }   /* :887-890 */

/* tanh_inplace (:1007-1021) */
void orc_tanh_inplace(float* x, int n) {
    for (int i = 0; i < n; i++) x[i] = i < body_len(n) ? lane_tanhf(x[i]) : portable_tanhf(x[i]);
}

/* sigmoid_inplace (:1023-1038) */
void orc_sigmoid_inplace(float* x, int n) {
    for (int i = 0; i < n; i++) x[i] = i < body_len(n) ? orc_lane_sigmoidf(x[i]) : portable_sigmoidf(x[i]);
}

/* sigmoid_add_into (:1040-1056): sigmoid(base + offset) */
void orc_sigmoid_add_into(float* out, const float* base, const float* offset, int n) {
    for (int i = 0; i < n; i++) {
        const float v = base[i] + offset[i];
        out[i] = i < body_len(n) ? orc_lane_sigmoidf(v) : portable_sigmoidf(v);
    }
}

/* decay_sigmoid_into (:1082-1101): exp(-0.606531 * sigmoid(base + offset)) */
void orc_decay_sigmoid_into(float* out, const float* base, const float* offset, int n) {
    for (int i = 0; i < n; i++) {
        const float v = base[i] + offset[i];
        out[i] = i < body_len(n) ? orc_lane_expf(-0.606531f * orc_lane_sigmoidf(v))
                                 : orc_expf(-0.606531f * portable_sigmoidf(v));
    }
}

/* sigmoid_mix_inplace (:1128-1147): v += (v_first - v) * sigmoid(base + offset) */
void orc_sigmoid_mix_inplace(float* v, const float* v_first, const float* base, const float* offset, int n) {
    for (int i = 0; i < n; i++) {
        const float x = base[i] + offset[i];
        const float mix = i < body_len(n) ? orc_lane_sigmoidf(x) : portable_sigmoidf(x);
        v[i] += (v_first[i] - v[i]) * mix;
    }
}

/* group_norm_into (:1400-1414). */
void orc_group_norm_into(float* out, const float* x, int groups, const float* w, const float* b, int n, float eps) {
    int gs = n / groups;
    for (int g = 0; g < groups; g++) {
        const float* s = x + g * gs;
        float sum = 0.0f;
        for (int i = 0; i < gs; i++) sum += s[i];
        float mean = sum / (float)gs;
        float vs = 0.0f;
        for (int i = 0; i < gs; i++) vs += (s[i] - mean) * (s[i] - mean);
        float inv_std = 1.0f / sqrtf(vs / (float)gs + eps);
        for (int i = g * gs; i < (g + 1) * gs; i++) out[i] = (x[i] - mean) * inv_std * w[i] + b[i];
    }
}

/* l2_normalize_per_head_inplace (:1416-1424). */
void orc_l2_normalize_per_head(float* x, int heads, int hs) {
    for (int h = 0; h < heads; h++) {
        float* s = x + h * hs;
        float sq = 0.0f;
        for (int i = 0; i < hs; i++) sq += s[i] * s[i];
        float norm = sqrtf(sq);
        float inv = norm > 1e-12f ? 1.0f / norm : 0.0f;
        for (int i = 0; i < hs; i++) s[i] *= inv;
    }
}

/* mat_vec_mul_small_into (:1892-1898): out[i] = sequential sum over j of a[i][j]*v[j]. */
void orc_mat_vec_small(float* out, const float* a, const float* v, int n) {
    for (int i = 0; i < n; i++) {
        float sum = 0.0f;
        for (int j = 0; j < n; j++) sum += a[i * n + j] * v[j];
        out[i] = sum;
    }
}

/* WKV-7 of one head (model.rs:869-891): with kk_a = kk*a and neg_kk = -kk,
 * t = S·neg_kk; S[i][j] = S[i][j]*w[j] + t[i]*kk_a[j] + v[i]*kmod[j]; out = S·r.
 * `tmp` holds 3n floats. */
void orc_wkv_head(float* S, int n, const float* r, const float* w, const float* kk, const float* a,
                  const float* v, const float* kmod, float* out, float* tmp) {
    float *kka = tmp, *negkk = tmp + n, *t = tmp + 2 * n;
    for (int j = 0; j < n; j++) kka[j] = kk[j] * a[j];
    for (int j = 0; j < n; j++) negkk[j] = -kk[j];
    orc_mat_vec_small(t, S, negkk, n);
    for (int i = 0; i < n; i++)
        for (int j = 0; j < n; j++) {
            const float sab = t[i] * kka[j];  /* outer_product_into (:1869-1877) */
            S[i * n + j] = S[i * n + j] * w[j] + sab + v[i] * kmod[j];
        }
    orc_mat_vec_small(out, S, r, n);
}

/* f32 mat_vec_mul_into (:1602-1705): one dot_avx2_order per row. */
static void matvec_f32(float* out, const float* m, int rows, int cols, const float* v) {
    for (int r = 0; r < rows; r++) out[r] = orc_dot_f32(m + (size_t)r * cols, v, cols);
}

/* quantize_vec_i8_into (tensor.rs:1791-1800): one scale for the whole vector, amax / 127
 * (1 for a vector without a nonzero magnitude; NaNs never raise amax), then
 * q = clamp(round(v * (1 / scale)), -127, 127) with Rust's round (half away from zero, as
 * C's roundf) and its saturating `as i8` (NaN -> 0). */
float orc_quantize_vec_i8(const float* v, int n, int8_t* q) {
    float amax = 0.0f;
    for (int i = 0; i < n; i++) {
        const float a = fabsf(v[i]);
        if (a > amax) amax = a;
    }
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    for (int i = 0; i < n; i++) {
        float t = roundf(v[i] * inv);
        if (t < -127.0f) t = -127.0f;
        if (t > 127.0f) t = 127.0f;
        q[i] = t != t ? 0 : (int8_t)t;
    }
    return scale;
}

/* q8_mat_vec_mul_scalar_into (tensor.rs:1838-1866): per row the exact int32 sum of
 * q[r][c] * vq[c], then (float)sum * (scale[r] * v_scale).  The reference's VNNI and AVX2
 * kernels (:238-330) reach the same integer sums, so every dispatch gives these bits. */
void orc_q8_matvec_a8(const int8_t* q, const float* scales, int rows, int cols, const int8_t* vq, float v_scale,
                      float* out) {
    for (int r = 0; r < rows; r++) {
        const int8_t* qr = q + (size_t)r * cols;
        int32_t s = 0;
        for (int c = 0; c < cols; c++) s += (int32_t)qr[c] * (int32_t)vq[c];
        out[r] = (float)s * (scales[r] * v_scale);
    }
}

/* ---- load ---- */

static void layer_free(RLayer* L) {
    float** vecs[] = {&L->ln1_w, &L->ln1_b, &L->ln2_w, &L->ln2_b, &L->x_r, &L->x_w, &L->x_k, &L->x_v,
                      &L->x_a, &L->x_g, &L->w0, &L->w1, &L->w2, &L->a0, &L->a1, &L->a2, &L->v0, &L->v1,
                      &L->v2, &L->g1, &L->g2, &L->k_k, &L->k_a, &L->r_k, &L->ln_x_w, &L->ln_x_b, &L->ffn_x_k};
    for (size_t i = 0; i < sizeof(vecs) / sizeof(vecs[0]); i++) { free(*vecs[i]); *vecs[i] = NULL; }
    mat_free(&L->r); mat_free(&L->k); mat_free(&L->v); mat_free(&L->o);
    mat_free(&L->fk); mat_free(&L->fv);
}

void orc_rwkv_free(OrcRwkv* m) {
    if (!m) return;
    if (m->layers) for (uint32_t i = 0; i < m->nl; i++) layer_free(&m->layers[i]);
    free(m->layers);
    free(m->emb); free(m->ln_out_w); free(m->ln_out_b);
    mat_free(&m->head);
    free(m->x_att); free(m->wkv); free(m->x_ffn); free(m->v_first); free(m->since);
    free(m);
}

OrcRwkv* orc_rwkv_load(const char* path, int profile) {
    if ((profile & 3) == 3) return NULL;
    if ((profile & ORC_PROFILE_W8A8) && (profile & 3) != ORC_PROFILE_Q8_ROW) return NULL;  /* per-row only */
    FILE* f = fopen(path, "rb");
    if (!f) return NULL;
    uint32_t h[16];
    if (fread(h, 4, 16, f) != 16 || h[0] != RWKV_MAGIC || h[1] != RWKV_VERSION || h[2] != RWKV_MODEL ||
        h[4] != h[5] * h[6] || h[4] == 0 || h[7] == 0 || h[3] == 0) {
        fclose(f);
        return NULL;
    }
    OrcRwkv* m = (OrcRwkv*)calloc(1, sizeof(OrcRwkv));
    m->vocab = h[3]; m->d = h[4]; m->h = h[5]; m->n = h[6]; m->nl = h[7]; m->f = h[8];
    m->rw = h[9]; m->ra = h[10]; m->rv = h[11]; m->rg = h[12]; m->g1k = h[13] & 1;
    m->profile = profile;
    const int quant = (profile & 3) != 0;
    const int group = (profile & 3) == 1 ? 64 : 0;  /* 0: one scale per row */
    const size_t d = m->d, ff = m->f;
    int ok = 1;
#define RD(p, cnt) do { if (ok && !((p) = read_f32(f, (cnt)))) ok = 0; } while (0)
#define RM(mat, rows, cols) do { float* t_ = NULL; RD(t_, (size_t)(rows) * (cols)); \
        if (ok && mat_make(&(mat), t_, (int)(rows), (int)(cols), quant, group ? group : (int)(cols))) ok = 0; } while (0)
    RD(m->emb, (size_t)m->vocab * d);
    m->layers = (RLayer*)calloc(m->nl, sizeof(RLayer));
    for (uint32_t i = 0; ok && i < m->nl; i++) {
        RLayer* L = &m->layers[i];
        RD(L->ln1_w, d); RD(L->ln1_b, d); RD(L->ln2_w, d); RD(L->ln2_b, d);
        RD(L->x_r, d); RD(L->x_w, d); RD(L->x_k, d); RD(L->x_v, d); RD(L->x_a, d); RD(L->x_g, d);
        RD(L->w0, d); RD(L->w1, m->rw * d); RD(L->w2, d * m->rw);
        RD(L->a0, d); RD(L->a1, m->ra * d); RD(L->a2, d * m->ra);
        RD(L->v0, d); RD(L->v1, m->rv * d); RD(L->v2, d * m->rv);
        RD(L->g1, m->rg * d); RD(L->g2, d * m->rg);
        RD(L->k_k, d); RD(L->k_a, d); RD(L->r_k, d);
        RM(L->r, d, d); RM(L->k, d, d); RM(L->v, d, d); RM(L->o, d, d);
        RD(L->ln_x_w, d); RD(L->ln_x_b, d); RD(L->ffn_x_k, d);
        RM(L->fk, ff, d); RM(L->fv, d, ff);
    }
    RD(m->ln_out_w, d); RD(m->ln_out_b, d);
    RM(m->head, m->vocab, d);
#undef RD
#undef RM
    if (ok) {
        char extra;
        ok = fread(&extra, 1, 1, f) == 0;  /* the body must end exactly */
    }
    fclose(f);
    if (!ok) { orc_rwkv_free(m); return NULL; }
    return m;
}

void orc_rwkv_dims(const OrcRwkv* m, uint32_t out[11]) {
    uint32_t v[11] = {m->vocab, m->d, m->h, m->n, m->nl, m->f, m->rw, m->ra, m->rv, m->rg, m->g1k};
    memcpy(out, v, sizeof(v));
}

static size_t wkv_len(const OrcRwkv* m) { return (size_t)m->h * m->n * m->n; }

int orc_rwkv_pool_init(OrcRwkv* m, uint32_t cap) {
    free(m->x_att); free(m->wkv); free(m->x_ffn); free(m->v_first); free(m->since);
    m->cap = cap;
    m->x_att = (float*)calloc((size_t)cap * m->nl * m->d, sizeof(float));
    m->wkv = (float*)calloc((size_t)cap * m->nl * wkv_len(m), sizeof(float));
    m->x_ffn = (float*)calloc((size_t)cap * m->nl * m->d, sizeof(float));
    m->v_first = (float*)calloc((size_t)cap * m->d, sizeof(float));
    m->since = (uint64_t*)calloc(cap, sizeof(uint64_t));
    return (m->x_att && m->wkv && m->x_ffn && m->v_first && m->since) ? 0 : -1;
}

/* Rwkv7State::reset (model.rs:135-140). */
static void reset_slot(OrcRwkv* m, uint32_t s) {
    memset(m->x_att + (size_t)s * m->nl * m->d, 0, sizeof(float) * m->nl * m->d);
    memset(m->wkv + (size_t)s * m->nl * wkv_len(m), 0, sizeof(float) * m->nl * wkv_len(m));
    memset(m->x_ffn + (size_t)s * m->nl * m->d, 0, sizeof(float) * m->nl * m->d);
    memset(m->v_first + (size_t)s * m->d, 0, sizeof(float) * m->d);
    m->since[s] = 0;
}

int orc_rwkv_reset(OrcRwkv* m, const uint32_t* slots, uint32_t n) {
    if (!slots) { for (uint32_t s = 0; s < m->cap; s++) reset_slot(m, s); return 0; }
    for (uint32_t i = 0; i < n; i++) if (slots[i] >= m->cap) return -1;
    for (uint32_t i = 0; i < n; i++) reset_slot(m, slots[i]);
    return 0;
}

void orc_rwkv_set_reset_every(OrcRwkv* m, uint64_t every) { m->reset_every = every; }

int orc_rwkv_get_state(const OrcRwkv* m, uint32_t slot, uint32_t layer, float* x_att, float* wkv, float* x_ffn) {
    if (slot >= m->cap || layer >= m->nl) return -1;
    const size_t d = m->d, w = wkv_len(m);
    if (x_att) memcpy(x_att, m->x_att + ((size_t)slot * m->nl + layer) * d, sizeof(float) * d);
    if (wkv) memcpy(wkv, m->wkv + ((size_t)slot * m->nl + layer) * w, sizeof(float) * w);
    if (x_ffn) memcpy(x_ffn, m->x_ffn + ((size_t)slot * m->nl + layer) * d, sizeof(float) * d);
    return 0;
}

/* ---- the step ---- */

typedef struct {
    float *x, *ln, *xx, *xr, *xw, *xk, *xv, *xa, *xg, *r, *k, *v, *w, *a, *kk, *kmod, *vout;
    float *outv, *outn, *g, *lorad, *lora, *tm, *cm, *fproj, *fact, *kka, *negkk, *outh;
    int8_t* vq;         /* the quantized input of a W8A8 projection (max(d, d_ffn)) */
} Scratch;

/* QuantMatrix::mat_vec_mul_into (quant.rs:321-330) of a quantized matrix: the W8A8 path
 * with profile bit 5 (q8_mat_vec_mul_into, tensor.rs:1819-1836), else the weight-only one. */
static void proj(const OrcRwkv* m, const Mat* w, const float* v, float* out, int8_t* vq) {
    if (m->profile & ORC_PROFILE_W8A8) {
        const float vs = orc_quantize_vec_i8(v, w->cols, vq);
        orc_q8_matvec_a8(w->q, w->sc, w->rows, w->cols, vq, vs, out);
    } else {
        mat_rows(w, 0, w->rows, v, out);
    }
}

/* time_mixing_scratch (model.rs:802-916) for one stream. */
static void time_mixing(const OrcRwkv* m, const RLayer* L, int layer, Scratch* s, const float* x_prev,
                        const float* v_first, float* S) {
    const int d = (int)m->d, H = (int)m->h, N = (int)m->n;
    /* Step 1: token shift (sub_into :739-741, add_scaled_into :747-751). */
    for (int i = 0; i < d; i++) s->xx[i] = x_prev[i] - s->ln[i];
    for (int i = 0; i < d; i++) {
        s->xr[i] = s->ln[i] + s->xx[i] * L->x_r[i];
        s->xw[i] = s->ln[i] + s->xx[i] * L->x_w[i];
        s->xk[i] = s->ln[i] + s->xx[i] * L->x_k[i];
        s->xv[i] = s->ln[i] + s->xx[i] * L->x_v[i];
        s->xa[i] = s->ln[i] + s->xx[i] * L->x_a[i];
        s->xg[i] = s->ln[i] + s->xx[i] * L->x_g[i];
    }
    /* Step 2: projections. */
    proj(m, &L->r, s->xr, s->r, s->vq);
    proj(m, &L->k, s->xk, s->k, s->vq);
    proj(m, &L->v, s->xv, s->v, s->vq);
    /* Step 3: decay = exp(-0.606531 * sigmoid(w0 + w2·tanh(w1·xw))). */
    const int rw = (int)m->rw, ra = (int)m->ra, rv = (int)m->rv, rg = (int)m->rg;
    matvec_f32(s->lora, L->w1, rw, d, s->xw);
    orc_tanh_inplace(s->lora, rw);
    matvec_f32(s->lorad, L->w2, d, rw, s->lora);
    orc_decay_sigmoid_into(s->w, L->w0, s->lorad, d);
    /* Step 4: a = sigmoid(a0 + a2·(a1·xa)). */
    matvec_f32(s->lora, L->a1, ra, d, s->xa);
    matvec_f32(s->lorad, L->a2, d, ra, s->lora);
    orc_sigmoid_add_into(s->a, L->a0, s->lorad, d);
    /* Step 5: g = g2·sigmoid(g1·xg). */
    matvec_f32(s->lora, L->g1, rg, d, s->xg);
    orc_sigmoid_inplace(s->lora, rg);
    matvec_f32(s->g, L->g2, d, rg, s->lora);
    /* Step 6: kk = l2norm_per_head(k * k_k) (mul_into :753-755). */
    for (int i = 0; i < d; i++) s->kk[i] = s->k[i] * L->k_k[i];
    orc_l2_normalize_per_head(s->kk, H, N);
    /* Step 7 */
    for (int i = 0; i < d; i++) s->kmod[i] = s->k[i] * (1.0f + (s->a[i] - 1.0f) * L->k_a[i]);
    /* Step 8: v_out = v, mixed towards v_first from the second layer on. */
    memcpy(s->vout, s->v, sizeof(float) * d);
    if (layer != 0) {
        matvec_f32(s->lora, L->v1, rv, d, s->xv);
        matvec_f32(s->lorad, L->v2, d, rv, s->lora);
        orc_sigmoid_mix_inplace(s->vout, v_first, L->v0, s->lorad, d);
    }
    /* Step 9: WKV-7 per head. */
    for (int hh = 0; hh < H; hh++) {
        const int hd = hh * N;
        orc_wkv_head(S + (size_t)hh * N * N, N, s->r + hd, s->w + hd, s->kk + hd, s->a + hd, s->vout + hd,
                     s->kmod + hd, s->outv + hd, s->kka);
    }
    /* Step 10: GroupNorm, eps 64e-5. */
    orc_group_norm_into(s->outn, s->outv, H, L->ln_x_w, L->ln_x_b, d, 64e-5f);
    /* Step 11: bonus (r * k * r_k summed per head) * v_out. */
    const float* ksrc = m->g1k ? s->kmod : s->k;
    for (int hh = 0; hh < H; hh++) {
        const int hd = hh * N;
        float bonus = 0.0f;
        for (int j = 0; j < N; j++) bonus += s->r[hd + j] * ksrc[hd + j] * L->r_k[hd + j];
        for (int j = 0; j < N; j++) s->outn[hd + j] += bonus * s->vout[hd + j];
    }
    /* Step 12: gate and output projection. */
    for (int i = 0; i < d; i++) s->xx[i] = s->outn[i] * s->g[i];
    proj(m, &L->o, s->xx, s->tm, s->vq);
}

/* channel_mixing_scratch (model.rs:919-925; squared_relu_into tensor.rs:1386-1388). */
static void channel_mixing(const OrcRwkv* m, const RLayer* L, Scratch* s, const float* x_prev) {
    const int d = (int)m->d, ff = (int)m->f;
    for (int i = 0; i < d; i++) s->xx[i] = x_prev[i] - s->ln[i];
    for (int i = 0; i < d; i++) s->xr[i] = s->ln[i] + s->xx[i] * L->ffn_x_k[i];
    proj(m, &L->fk, s->xr, s->fproj, s->vq);
    for (int i = 0; i < ff; i++) {
        const float r = s->fproj[i] > 0.0f ? s->fproj[i] : 0.0f;  /* f32::max(x, 0): NaN -> 0 */
        s->fact[i] = r * r;
    }
    proj(m, &L->fv, s->fact, s->cm, s->vq);
}

typedef struct {
    OrcRwkv* m;
    const uint32_t* slots;
    const uint32_t* tokens;
    float* out;
} StepJob;

/* forward_into (model.rs:643-698) for stream b. */
static void stream_step(void* ctx, int b) {
    StepJob* j = (StepJob*)ctx;
    OrcRwkv* m = j->m;
    const uint32_t slot = j->slots[b];
    const int d = (int)m->d, N = (int)m->n, ff = (int)m->f;
    int lmax = (int)m->rw;
    if ((int)m->ra > lmax) lmax = (int)m->ra;
    if ((int)m->rv > lmax) lmax = (int)m->rv;
    if ((int)m->rg > lmax) lmax = (int)m->rg;
    const size_t dsz = (size_t)d;
    float* buf = (float*)calloc(dsz * 24 + (size_t)lmax + 2 * (size_t)ff + 3 * (size_t)N, sizeof(float));  /* kka: 3N */
    int8_t* vq = (int8_t*)malloc(dsz > (size_t)ff ? dsz : (size_t)ff);
    if (!buf || !vq) { free(buf); free(vq); return; }
    Scratch s;
    float* p = buf;
    float** dvecs[] = {&s.x, &s.ln, &s.xx, &s.xr, &s.xw, &s.xk, &s.xv, &s.xa, &s.xg, &s.r, &s.k, &s.v, &s.w,
                       &s.a, &s.kk, &s.kmod, &s.vout, &s.outv, &s.outn, &s.g, &s.lorad, &s.tm, &s.cm};
    for (size_t i = 0; i < sizeof(dvecs) / sizeof(dvecs[0]); i++) { *dvecs[i] = p; p += dsz; }
    s.lora = p; p += lmax;
    s.fproj = p; p += ff;
    s.fact = p; p += ff;
    s.kka = p; p += N;
    s.negkk = p; p += N;
    s.outh = p;
    s.vq = vq;

    memcpy(s.x, m->emb + (size_t)j->tokens[b] * d, sizeof(float) * d);
    float* vfirst = m->v_first + (size_t)slot * d;
    for (uint32_t i = 0; i < m->nl; i++) {
        const RLayer* L = &m->layers[i];
        float* xa = m->x_att + ((size_t)slot * m->nl + i) * d;
        float* xf = m->x_ffn + ((size_t)slot * m->nl + i) * d;
        float* S = m->wkv + ((size_t)slot * m->nl + i) * wkv_len(m);
        orc_layer_norm(s.ln, s.x, L->ln1_w, L->ln1_b, d, 1e-5f);  /* layer_norm_into, tensor.rs:1390-1398 */
        time_mixing(m, L, (int)i, &s, xa, vfirst, S);
        memcpy(xa, s.ln, sizeof(float) * d);
        if (i == 0) memcpy(vfirst, s.v, sizeof(float) * d);
        for (int c = 0; c < d; c++) s.x[c] += s.tm[c];
        orc_layer_norm(s.ln, s.x, L->ln2_w, L->ln2_b, d, 1e-5f);
        channel_mixing(m, L, &s, xf);
        memcpy(xf, s.ln, sizeof(float) * d);
        for (int c = 0; c < d; c++) s.x[c] += s.cm[c];
    }
    orc_layer_norm(s.ln, s.x, m->ln_out_w, m->ln_out_b, d, 1e-5f);
    proj(m, &m->head, s.ln, j->out + (size_t)b * m->vocab, s.vq);
    free(buf);
    free(vq);
}

int orc_rwkv_forward(OrcRwkv* m, uint32_t n, const uint32_t* slots, const uint32_t* tokens, float* out) {
    if (n == 0) return 0;
    if (!m->cap || n > m->cap) return -1;
    for (uint32_t b = 0; b < n; b++) {
        if (slots[b] >= m->cap || tokens[b] >= m->vocab) return -1;
        for (uint32_t c = 0; c < b; c++) if (slots[c] == slots[b]) return -1;
    }
    /* Periodic reset before the (k*every + 1)-th forward of a slot, as the host's
     * PluginState::tick does (plugin_backend/model.rs:44-49). */
    for (uint32_t b = 0; b < n; b++) {
        if (m->reset_every && m->since[slots[b]] >= m->reset_every) reset_slot(m, slots[b]);
        m->since[slots[b]]++;
    }
    StepJob j = {m, slots, tokens, out};
    pool_run((int)n, stream_step, &j);
    return 0;
}
