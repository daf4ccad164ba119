/* mamba_oracle.c — CPU restatement of redukt's Mamba-1 CPU step.
 *
 * TEST INFRASTRUCTURE ONLY: the parity oracle and the timed CPU baseline ("port").
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Numeric contract: the reference's "Plain" kernel family (numeric contracts 0/1,
 * src/domain/gemv.rs:13-21): IEEE f32, separate multiply and add, no contraction
 * (built with -ffp-contract=off), the reference's own portable exp/ln
 * (src/domain/tensor.rs:757-915), and the reference's accumulation orders.  With
 * ORC_PROFILE_FMA the GEMVs take numeric contract 2 instead (the "Fma" kernel family,
 * src/domain/gemv_fma.rs:1-26): the same orders, each acc + w*x one fused multiply-add
 * (C99 fmaf, correctly rounded like the reference's fma_f32, gemv_fma.rs:61-96).  Every
 * function cites the reference code it restates.  Nothing here is shared with the
 * HIP product library.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "internal.h"
#include "oracle.h"
#include "pool.h"

#if defined(__x86_64__) && defined(__GNUC__) && !defined(__clang__)
#define VEC_CLONES __attribute__((target_clones("avx2", "default")))
#else
#define VEC_CLONES
#endif

/* ====================================================================
 * Portable transcendentals — src/domain/tensor.rs:757-915
 * ==================================================================== */

static inline float f_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* tensor.rs:912-915: round half to even via the 2^23 trick. */
static inline float roundeven_f(float x) {
    const float MAGIC = 8388608.0f;
    return x >= 0.0f ? (x + MAGIC) - MAGIC : (x - MAGIC) + MAGIC;
}

/* tensor.rs:765-794: Cephes degree-5 polynomial with range reduction. */
float orc_expf(float x) {
    const float LOG2E = 1.44269504088896341f;
    const float LN2_HI = 6.93145751953125E-1f;
    const float LN2_LO = 1.42860682030941723212E-6f;
    const float EXP_LO = -87.3365447505531f;
    const float EXP_HI = 88.3762626647949f;
    const float P0 = 1.9875691500E-4f, P1 = 1.3981999507E-3f, P2 = 8.3334519073E-3f;
    const float P3 = 4.1665795894E-2f, P4 = 1.6666665459E-1f, P5 = 5.0000001201E-1f;
    x = x < EXP_LO ? EXP_LO : (x > EXP_HI ? EXP_HI : x);
    float fx = x * LOG2E;
    float nf = roundeven_f(fx);
    int32_t n = isnan(nf) ? 0 : (int32_t)nf; /* Rust `as i32` maps NaN to 0 */
    float r = (x - nf * LN2_HI) - nf * LN2_LO;
    float r2 = r * r;
    float y = P0;
    y = y * r + P1;
    y = y * r + P2;
    y = y * r + P3;
    y = y * r + P4;
    y = y * r + P5;
    y = (y * r2 + r) + 1.0f;
    float pow2n = f_from_bits(((uint32_t)(n + 127)) << 23);
    return y * pow2n;
}

/* tensor.rs:799-837: musl/FreeBSD logf. */
float orc_lnf(float x) {
    const float LN2_HI = 6.9313812256e-01f, LN2_LO = 9.0580006145e-06f;
    const float LG1 = 0.66666662693f, LG2 = 0.40000972152f, LG3 = 0.28498786688f, LG4 = 0.24279078841f;
    uint32_t ix = bits_of(x);
    int32_t k = 0;
    if (ix < 0x00800000u || (ix >> 31) != 0) {
        if ((uint32_t)(ix << 1) == 0) return -INFINITY;
        if ((ix >> 31) != 0) return NAN;
        k -= 25;
        ix = bits_of(x * f_from_bits(0x4c000000u));
    } else if (ix >= 0x7f800000u) {
        return x;
    } else if (ix == 0x3f800000u) {
        return 0.0f;
    }
    ix = ix + (0x3f800000u - 0x3f3504f3u);
    k += (int32_t)(ix >> 23) - 0x7f;
    ix = (ix & 0x007fffffu) + 0x3f3504f3u;
    float xn = f_from_bits(ix);
    float f = xn - 1.0f;
    float s = f / (2.0f + f);
    float dk = (float)k;
    float z = s * s;
    float w = z * z;
    float t1 = w * (LG2 + w * LG4);
    float t2 = z * (LG1 + w * LG3);
    float r = t2 + t1;
    float hfsq = 0.5f * f * f;
    return s * (hfsq + r) + dk * LN2_LO - hfsq + f + dk * LN2_HI;
}

/* tensor.rs:877-879: one lane of fast_exp_ps (a NaN lane is clamped to EXP_LO). */
float orc_lane_expf(float x) { return orc_expf(isnan(x) ? -87.3365447505531f : x); }
/* tensor.rs:883-885 */
float orc_lane_sigmoidf(float x) { return 1.0f / (1.0f + orc_lane_expf(0.0f - x)); }
#define lane_sigmoidf orc_lane_sigmoidf
/* tensor.rs:841-843 */
float orc_sigmoidf(float x) { return 1.0f / (1.0f + orc_expf(-x)); }
/* tensor.rs:853-855 */
static inline float portable_silu(float x) { return x * orc_sigmoidf(x); }
/* tensor.rs:859-861 */
float orc_softplus(float x) { return x > 20.0f ? x : orc_lnf(1.0f + orc_expf(x)); }

/* tensor.rs:1917-1933: max, portable exp, sequential sum, division. */
void orc_softmax_into(const float* logits, float* out, int n) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) mx = fmaxf(mx, logits[i]);
    if (mx == -INFINITY) {
        float u = 1.0f / (float)n;
        for (int i = 0; i < n; i++) out[i] = u;
        return;
    }
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        float e = orc_expf(logits[i] - mx);
        out[i] = e;
        sum += e;
    }
    float denom = fmaxf(sum, 1.1920929e-07f);
    for (int i = 0; i < n; i++) out[i] /= denom;
}

/* ====================================================================
 * GEMV orders — tensor.rs:1663-1705, gemv.rs:181-502
 * ==================================================================== */

/* tensor.rs:1666-1672 (hsum_f32_scalar) + 1680-1693 (dot_avx2_order): 8 lanes by column
 * residue from +0, ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)), then the sequential tail. */
VEC_CLONES float orc_dot_f32(const float* w, const float* v, int n) {
    int body = n / 8 * 8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int c = 0; c < body; c += 8)
        for (int l = 0; l < 8; l++) acc[l] += w[c + l] * v[c + l];
    float s0 = acc[0] + acc[4], s1 = acc[1] + acc[5], s2 = acc[2] + acc[6], s3 = acc[3] + acc[7];
    float s = (s0 + s2) + (s1 + s3);
    for (int c = body; c < n; c++) s += w[c] * v[c];
    return s;
}

/* gemv.rs:462-487 (hsum8_scalar, group_dot_scalar): same lane order on int8 weights. */
VEC_CLONES static float group_dot_q8(const int8_t* q, const float* v, int n) {
    int body = n / 8 * 8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int c = 0; c < body; c += 8)
        for (int l = 0; l < 8; l++) acc[l] += (float)q[c + l] * v[c + l];
    float s0 = acc[0] + acc[4], s1 = acc[1] + acc[5], s2 = acc[2] + acc[6], s3 = acc[3] + acc[7];
    float s = (s0 + s2) + (s1 + s3);
    for (int c = body; c < n; c++) s += (float)q[c] * v[c];
    return s;
}

/* gemv.rs:490-502: row = 0 + Σ_g dot_g * scale_g in group order. */
static float q8_row(const int8_t* q, const float* sc, int cols, int group, const float* v) {
    int gpr = cols / group;
    float row_sum = 0.0f;
    for (int g = 0; g < gpr; g++) row_sum += group_dot_q8(q + g * group, v + g * group, group) * sc[g];
    return row_sum;
}

/* gemv_fma.rs:98-112 (dot_fma_scalar): the lane order of orc_dot_f32 with every
 * acc + w*x one fused multiply-add, from +0; the horizontal sum with plain adds; the tail
 * by fused multiply-adds.  Q8 weights convert to f32 exactly (gemv_fma.rs:8-13). */
VEC_CLONES float orc_dot_f32_fma(const float* w, const float* v, int n) {
    int body = n / 8 * 8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int c = 0; c < body; c += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf(w[c + l], v[c + l], acc[l]);
    float s0 = acc[0] + acc[4], s1 = acc[1] + acc[5], s2 = acc[2] + acc[6], s3 = acc[3] + acc[7];
    float s = (s0 + s2) + (s1 + s3);
    for (int c = body; c < n; c++) s = fmaf(w[c], v[c], s);
    return s;
}

VEC_CLONES static float group_dot_q8_fma(const int8_t* q, const float* v, int n) {
    int body = n / 8 * 8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int c = 0; c < body; c += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf((float)q[c + l], v[c + l], acc[l]);
    float s0 = acc[0] + acc[4], s1 = acc[1] + acc[5], s2 = acc[2] + acc[6], s3 = acc[3] + acc[7];
    float s = (s0 + s2) + (s1 + s3);
    for (int c = body; c < n; c++) s = fmaf((float)q[c], v[c], s);
    return s;
}

/* gemv_fma.rs:121-134 (q8w_rows_fma_scalar): sum = fma(dot_g, scale_g, sum) from +0. */
static float q8_row_fma(const int8_t* q, const float* sc, int cols, int group, const float* v) {
    int gpr = cols / group;
    float row_sum = 0.0f;
    for (int g = 0; g < gpr; g++) row_sum = fmaf(group_dot_q8_fma(q + g * group, v + g * group, group), sc[g], row_sum);
    return row_sum;
}

/* gemv.rs:256-273: group rule, scale = amax/127 (1 if amax == 0), q = clamp(round(w/scale)). */
void orc_quantize(const float* w, int rows, int cols, int group, int8_t* q, float* scales, int* group_out) {
    if (!(group > 0 && group % 8 == 0 && cols % group == 0)) group = cols;
    size_t total = (size_t)rows * cols;
    size_t ngroups = total / (size_t)group;
    for (size_t gi = 0; gi < ngroups; gi++) {
        const float* wg = w + gi * group;
        float amax = 0.0f;
        for (int i = 0; i < group; i++) amax = fmaxf(amax, fabsf(wg[i]));
        float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        float inv = 1.0f / scale;
        for (int i = 0; i < group; i++) {
            float r = roundf(wg[i] * inv); /* Rust f32::round: half away from zero */
            r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
            q[gi * group + i] = isnan(r) ? 0 : (int8_t)r; /* Rust `as i8` maps NaN to 0 */
        }
        scales[gi] = scale;
    }
    if (group_out) *group_out = group;
}

void orc_gemv_f32(const float* w, int rows, int cols, const float* v, float* out) {
    for (int r = 0; r < rows; r++) out[r] = orc_dot_f32(w + (size_t)r * cols, v, cols);
}

void orc_gemv_q8(const int8_t* q, const float* scales, int rows, int cols, int group, const float* v, float* out) {
    int gpr = cols / group;
    for (int r = 0; r < rows; r++) out[r] = q8_row(q + (size_t)r * cols, scales + (size_t)r * gpr, cols, group, v);
}

void orc_gemv_f32_fma(const float* w, int rows, int cols, const float* v, float* out) {
    for (int r = 0; r < rows; r++) out[r] = orc_dot_f32_fma(w + (size_t)r * cols, v, cols);
}

void orc_gemv_q8_fma(const int8_t* q, const float* scales, int rows, int cols, int group, const float* v, float* out) {
    int gpr = cols / group;
    for (int r = 0; r < rows; r++) out[r] = q8_row_fma(q + (size_t)r * cols, scales + (size_t)r * gpr, cols, group, v);
}

/* ====================================================================
 * Norms and the selective scan — tensor.rs:900-908, 1283-1325, 1390-1398
 * ==================================================================== */

/* tensor.rs:900-908 */
void orc_rms_norm(float* x, const float* w, int n, float eps) {
    float sum_sq = 0.0f;
    for (int i = 0; i < n; i++) sum_sq += x[i] * x[i];
    float rms = sqrtf(sum_sq / (float)n + eps);
    float inv = 1.0f / rms;
    for (int i = 0; i < n; i++) x[i] = x[i] * inv * w[i];
}

/* tensor.rs:1390-1398 (two-pass) */
void orc_layer_norm(float* out, const float* x, const float* w, const float* b, int n, float eps) {
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += x[i];
    float mean = sum / (float)n;
    float vs = 0.0f;
    for (int i = 0; i < n; i++) vs += (x[i] - mean) * (x[i] - mean);
    float var = vs / (float)n;
    float inv_std = 1.0f / sqrtf(var + eps);
    for (int i = 0; i < n; i++) out[i] = (x[i] - mean) * inv_std * w[i] + b[i];
}

/* tensor.rs:1283 (DT_SPARSE_EPS), 1288-1294 (hsum_ssm_scalar), 1301-1325 (scalar twin of the
 * AVX2 scan): skip when |dt| < 1e-6, decay exp(0 - dt*exp(a_log)), s = da*s + (dt*x)*b,
 * y = ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)) over l[i] = s[i]c[i] + s[i+8]c[i+8], + d*x. */
void orc_ssm_d16(float* y, float* ss, const float* dt, const float* conv_out, const float* a_log,
                 const float* b, const float* c, const float* d_vec, int d_inner) {
    for (int j = 0; j < d_inner; j++) {
        float* st = ss + (size_t)j * 16;
        int skip = fabsf(dt[j]) < 1e-6f;
        if (!skip) {
            float dtx = dt[j] * conv_out[j];
            for (int n = 0; n < 16; n++) {
                float a = orc_lane_expf(a_log[(size_t)j * 16 + n]);
                float da = orc_lane_expf(0.0f - dt[j] * a);
                st[n] = da * st[n] + dtx * b[n];
            }
        }
        float l[8];
        for (int i = 0; i < 8; i++) l[i] = st[i] * c[i] + st[i + 8] * c[i + 8];
        float s0 = l[0] + l[4], s1 = l[1] + l[5], s2 = l[2] + l[6], s3 = l[3] + l[7];
        y[j] = ((s0 + s1) + (s2 + s3)) + d_vec[j] * conv_out[j];
    }
}

/* ====================================================================
 * Model — src/infrastructure/mamba/model.rs
 * ==================================================================== */

typedef struct {
    float *norm_w, *norm_b;
    Mat in_proj, x_proj, dt_proj, out_proj;
    float *conv_w, *conv_b, *dt_b, *a_log, *d_vec;
} Layer;

struct OrcMamba {
    uint32_t vocab, d, di, ds, dc, dr, nl, flags;
    int profile;
    Mat emb, head_own;
    Mat* head;
    Layer* layers;
    float *norm_f_w, *norm_f_b;
    /* slot pool */
    uint32_t cap;
    float* conv_st;     /* [slot][layer][di*(dc-1)] */
    float* ssm_st;      /* [slot][layer][di*16] */
    uint64_t* since;    /* forwards since the last reset, per slot */
    uint64_t reset_every;
    /* per-stream scratch (grown on demand) */
    uint32_t scratch_n;
    float *x, *normed, *xz, *conv_out, *zp, *dt, *y, *gated, *res;
};

void mat_free(Mat* m) { free(m->f); free(m->q); free(m->sc); memset(m, 0, sizeof(*m)); }

/* MambaMatrix::new (model.rs:64-69) and, with profile bit 2, the same recipe on x/dt_proj. */
int mat_make(Mat* m, float* data, int rows, int cols, int quant, int group) {
    m->rows = rows; m->cols = cols;
    if (!quant) { m->f = data; m->group = 0; return 0; }
    int g = group > 0 ? group : cols;
    if (!(g % 8 == 0 && cols % g == 0)) g = cols;
    m->q = (int8_t*)malloc((size_t)rows * cols);
    m->sc = (float*)malloc(sizeof(float) * ((size_t)rows * cols / g));
    if (!m->q || !m->sc) { free(data); return -1; }
    orc_quantize(data, rows, cols, g, m->q, m->sc, &m->group);
    free(data);
    return 0;
}

/* Row `row` into out: copy (F32) or q*scale per group (gemv.rs:285-295). */
void mat_row(const Mat* m, int row, float* out) {
    if (!m->group) { memcpy(out, m->f + (size_t)row * m->cols, sizeof(float) * m->cols); return; }
    int gpr = m->cols / m->group;
    const int8_t* q = m->q + (size_t)row * m->cols;
    const float* sc = m->sc + (size_t)row * gpr;
    for (int c = 0; c < m->cols; c++) out[c] = (float)q[c] * sc[c / m->group];
}

/* Rows [r0, r1) of out = M·v in the reference order (f32_rows / q8w_rows, or their
 * contract-2 twins f32_rows_fma_scalar / q8w_rows_fma_scalar, gemv_fma.rs:115-134). */
void mat_rows(const Mat* m, int r0, int r1, const float* v, float* out) {
    if (!m->group) {
        for (int r = r0; r < r1; r++)
            out[r] = m->fma ? orc_dot_f32_fma(m->f + (size_t)r * m->cols, v, m->cols)
                            : orc_dot_f32(m->f + (size_t)r * m->cols, v, m->cols);
    } else {
        int gpr = m->cols / m->group;
        for (int r = r0; r < r1; r++)
            out[r] = m->fma ? q8_row_fma(m->q + (size_t)r * m->cols, m->sc + (size_t)r * gpr, m->cols, m->group, v)
                            : q8_row(m->q + (size_t)r * m->cols, m->sc + (size_t)r * gpr, m->cols, m->group, v);
    }
}

float* read_f32(FILE* f, size_t count) {
    float* p = (float*)malloc(sizeof(float) * (count ? count : 1));
    if (!p) return NULL;
    if (fread(p, sizeof(float), count, f) != count) { free(p); return NULL; }
    return p;
}

void orc_mamba_free(OrcMamba* m) {
    if (!m) return;
    for (uint32_t i = 0; m->layers && i < m->nl; i++) {
        Layer* L = &m->layers[i];
        free(L->norm_w); free(L->norm_b); free(L->conv_w); free(L->conv_b);
        free(L->dt_b); free(L->a_log); free(L->d_vec);
        mat_free(&L->in_proj); mat_free(&L->x_proj); mat_free(&L->dt_proj); mat_free(&L->out_proj);
    }
    free(m->layers);
    mat_free(&m->emb);
    mat_free(&m->head_own);
    free(m->norm_f_w); free(m->norm_f_b);
    free(m->conv_st); free(m->ssm_st); free(m->since);
    free(m->x); free(m->normed); free(m->xz); free(m->conv_out); free(m->zp);
    free(m->dt); free(m->y); free(m->gated); free(m->res);
    free(m);
}

/* .rbin v1/v2 (scripts/convert-weights-gpu.py:43-53, 152-197): 11 LE u32 header, then f32
 * emb, per layer (norm_w, [norm_b], in_proj, conv_w, conv_b, x_proj, dt_w, dt_b, A_log, D,
 * out_proj), norm_f_w, [norm_f_b], [lm_head].  Header checks follow the plugin's
 * validate_header (plugins/redukt-gpu-cuda/mamba_cuda.cu:470-486); the CPU scan
 * additionally fixes d_state = 16 (tensor.rs ssm_recurrence_d16). */
OrcMamba* orc_mamba_load(const char* path, int profile, int* err) {
    *err = 4;
    FILE* f = fopen(path, "rb");
    if (!f) return NULL;
    uint32_t h[11];
    if (fread(h, 4, 11, f) != 11) { fclose(f); return NULL; }
    if (h[0] != 0x55504752u || (h[1] != 1 && h[1] != 2)) { fclose(f); return NULL; }
    if (!h[2] || !h[3] || !h[4] || !h[5] || !h[7] || !h[8] || h[6] < 2 || h[5] != 16) { fclose(f); return NULL; }
    if (h[1] == 2 && (h[10] > 1 || (h[10] == 0 && h[2] != 256))) { fclose(f); return NULL; }
    OrcMamba* m = (OrcMamba*)calloc(1, sizeof(OrcMamba));
    if (!m) { fclose(f); *err = 1; return NULL; }
    m->vocab = h[2]; m->d = h[3]; m->di = h[4]; m->ds = h[5]; m->dc = h[6]; m->dr = h[7];
    m->nl = h[8]; m->flags = h[9]; m->profile = profile;
    int quant = (profile & 3) != 0;
    int group = (profile & 3) == 1 ? 64 : 0;  /* 0 = per row */
    int qsmall = quant && (profile & ORC_PROFILE_Q8_SMALL);
    int nb = (m->flags & 1) != 0, uh = (m->flags & 2) != 0;
    size_t V = m->vocab, d = m->d, di = m->di, ds = m->ds, dc = m->dc, dr = m->dr, xr = dr + 2 * ds;
    float* t;
    int bad = 0;
    if (!(t = read_f32(f, V * d)) || mat_make(&m->emb, t, (int)V, (int)d, quant, group)) bad = 1;
    m->layers = (Layer*)calloc(m->nl, sizeof(Layer));
    if (!m->layers) bad = 1;
    for (uint32_t i = 0; !bad && i < m->nl; i++) {
        Layer* L = &m->layers[i];
        bad |= !(L->norm_w = read_f32(f, d));
        if (!bad && nb) bad |= !(L->norm_b = read_f32(f, d));
        if (!bad) bad |= !(t = read_f32(f, 2 * di * d)) || mat_make(&L->in_proj, t, (int)(2 * di), (int)d, quant, group);
        if (!bad) bad |= !(L->conv_w = read_f32(f, di * dc));
        if (!bad) bad |= !(L->conv_b = read_f32(f, di));
        if (!bad) bad |= !(t = read_f32(f, xr * di)) || mat_make(&L->x_proj, t, (int)xr, (int)di, qsmall, group);
        if (!bad) bad |= !(t = read_f32(f, di * dr)) || mat_make(&L->dt_proj, t, (int)di, (int)dr, qsmall, group);
        if (!bad) bad |= !(L->dt_b = read_f32(f, di));
        if (!bad) bad |= !(L->a_log = read_f32(f, di * ds));
        if (!bad) bad |= !(L->d_vec = read_f32(f, di));
        if (!bad) bad |= !(t = read_f32(f, d * di)) || mat_make(&L->out_proj, t, (int)d, (int)di, quant, group);
    }
    if (!bad) bad |= !(m->norm_f_w = read_f32(f, d));
    if (!bad && nb) bad |= !(m->norm_f_b = read_f32(f, d));
    if (!bad && uh) {
        bad |= !(t = read_f32(f, V * d)) || mat_make(&m->head_own, t, (int)V, (int)d, quant, group);
        m->head = &m->head_own;
    } else {
        m->head = &m->emb;
    }
    fclose(f);
    if (bad) { orc_mamba_free(m); return NULL; }
    /* MambaModel::set_kernel (model.rs:955-967): the kernel family of every GEMV (in_proj,
     * x_proj, dt_proj, out_proj, the head); the embedding lookup has no sum. */
    int fma = (profile & ORC_PROFILE_FMA) != 0;
    m->emb.fma = fma;
    m->head_own.fma = fma;
    for (uint32_t i = 0; i < m->nl; i++) {
        Layer* L = &m->layers[i];
        L->in_proj.fma = L->x_proj.fma = L->dt_proj.fma = L->out_proj.fma = fma;
    }
    *err = 0;
    return m;
}

void orc_mamba_dims(const OrcMamba* m, uint32_t out[8]) {
    out[0] = m->vocab; out[1] = m->d; out[2] = m->di; out[3] = m->ds;
    out[4] = m->dc; out[5] = m->dr; out[6] = m->nl; out[7] = m->flags;
}

static size_t conv_len(const OrcMamba* m) { return (size_t)m->di * (m->dc - 1); }
static size_t ssm_len(const OrcMamba* m) { return (size_t)m->di * 16; }

int orc_mamba_pool_init(OrcMamba* m, uint32_t cap) {
    free(m->conv_st); free(m->ssm_st); free(m->since);
    m->conv_st = NULL; m->ssm_st = NULL; m->since = NULL; m->cap = 0;
    if (cap == 0) return 0;
    m->conv_st = (float*)calloc((size_t)cap * m->nl * conv_len(m), sizeof(float));
    m->ssm_st = (float*)calloc((size_t)cap * m->nl * ssm_len(m), sizeof(float));
    m->since = (uint64_t*)calloc(cap, sizeof(uint64_t));
    if (!m->conv_st || !m->ssm_st || !m->since) return 1;
    m->cap = cap;
    return 0;
}

static void reset_slot(OrcMamba* m, uint32_t s) {
    memset(m->conv_st + (size_t)s * m->nl * conv_len(m), 0, sizeof(float) * m->nl * conv_len(m));
    memset(m->ssm_st + (size_t)s * m->nl * ssm_len(m), 0, sizeof(float) * m->nl * ssm_len(m));
    m->since[s] = 0;
}

/* MambaState::reset (model.rs:296-300) for the listed slots. */
int orc_mamba_reset(OrcMamba* m, const uint32_t* slots, uint32_t n) {
    if (!slots) { for (uint32_t s = 0; s < m->cap; s++) reset_slot(m, s); return 0; }
    for (uint32_t i = 0; i < n; i++) if (slots[i] >= m->cap) return 5;
    for (uint32_t i = 0; i < n; i++) reset_slot(m, slots[i]);
    return 0;
}

void orc_mamba_set_reset_every(OrcMamba* m, uint64_t every) { m->reset_every = every; }

static int grow_scratch(OrcMamba* m, uint32_t n) {
    if (n <= m->scratch_n) return 0;
    size_t d = m->d, di = m->di, xr = m->dr + 2 * m->ds;
#define GROW(p, len) do { free(m->p); m->p = (float*)calloc((size_t)n * (len), sizeof(float)); if (!m->p) return 1; } while (0)
    GROW(x, d); GROW(normed, d); GROW(xz, 2 * di); GROW(conv_out, di); GROW(zp, xr);
    GROW(dt, di); GROW(y, di); GROW(gated, di); GROW(res, d);
#undef GROW
    m->scratch_n = n;
    return 0;
}

/* ---- pooled phases ---- */

typedef struct {
    OrcMamba* m;
    const Mat* w;
    const float* x; size_t ldx;   /* stream b's input at x + b*ldx */
    float* y; size_t ldy;
    uint32_t n;
    int rpb;                      /* rows per block */
} GemvJob;

/* gemv_*_multi (gemv.rs:213-236, 319-337): one row block, every stream; per (stream,row)
 * the single-stream kernel's arithmetic, so the result is independent of n and threads. */
static void gemv_block(void* ctx, int b) {
    GemvJob* j = (GemvJob*)ctx;
    int r0 = b * j->rpb, r1 = r0 + j->rpb;
    if (r1 > j->w->rows) r1 = j->w->rows;
    for (uint32_t s = 0; s < j->n; s++) mat_rows(j->w, r0, r1, j->x + s * j->ldx, j->y + s * j->ldy);
}

static void gemv_multi(OrcMamba* m, const Mat* w, const float* x, size_t ldx, float* y, size_t ldy, uint32_t n) {
    int threads = orc_get_threads();
    int rows = w->rows;
    int rpb = rows / (threads * 8 > 0 ? threads * 8 : 1);
    if (rpb < 4) rpb = 4;
    rpb = (rpb + 3) / 4 * 4;
    GemvJob j = { m, w, x, ldx, y, ldy, n, rpb };
    pool_run((rows + rpb - 1) / rpb, gemv_block, &j);
}

typedef struct {
    OrcMamba* m;
    const Layer* L;
    uint32_t li, n;
    const uint32_t* slots;
    int nblk;                     /* channel blocks per stream */
} PhaseJob;

/* conv_silu_block (model.rs:134-153) + silu_inplace on the block (tensor.rs:1197-1211):
 * 8-aligned body with the lane sigmoid, portable tail. */
static void conv_block(void* ctx, int u) {
    PhaseJob* j = (PhaseJob*)ctx;
    OrcMamba* m = j->m;
    const Layer* L = j->L;
    uint32_t s = (uint32_t)u / j->nblk, bi = (uint32_t)u % j->nblk;
    size_t di = m->di, dc = m->dc;
    size_t j0 = (size_t)bi * 256, j1 = j0 + 256 > di ? di : j0 + 256;
    float* cs = m->conv_st + ((size_t)j->slots[s] * m->nl + j->li) * conv_len(m);
    const float* x = m->xz + s * 2 * di;
    float* out = m->conv_out + s * di;
    for (size_t jj = j0; jj < j1; jj++) {
        float* st = cs + jj * (dc - 1);
        const float* w = L->conv_w + jj * dc;
        float val = 0.0f;
        for (size_t k = 0; k < dc - 1; k++) val += st[k] * w[k];
        val += x[jj] * w[dc - 1];
        val += L->conv_b[jj];
        for (size_t k = 0; k + 2 < dc; k++) st[k] = st[k + 1];
        st[dc - 2] = x[jj];
        out[jj] = val;
    }
    size_t len = j1 - j0, body = len / 8 * 8;
    for (size_t i = 0; i < body; i++) out[j0 + i] *= lane_sigmoidf(out[j0 + i]);
    for (size_t i = body; i < len; i++) out[j0 + i] = portable_silu(out[j0 + i]);
}

/* scan_block (model.rs:174-190): dt_proj rows of the block, softplus(dt + bias), the d16
 * scan, then gated_silu_mul on the block (tensor.rs:1239-1243). */
static void scan_block(void* ctx, int u) {
    PhaseJob* j = (PhaseJob*)ctx;
    OrcMamba* m = j->m;
    const Layer* L = j->L;
    uint32_t s = (uint32_t)u / j->nblk, bi = (uint32_t)u % j->nblk;
    size_t di = m->di, dr = m->dr, ds = m->ds, xr = dr + 2 * ds;
    size_t j0 = (size_t)bi * 64, j1 = j0 + 64 > di ? di : j0 + 64;
    const float* zp = m->zp + s * xr;
    float* dt = m->dt + s * di;
    mat_rows(&L->dt_proj, (int)j0, (int)j1, zp, dt);
    for (size_t jj = j0; jj < j1; jj++) dt[jj] = orc_softplus(dt[jj] + L->dt_b[jj]);
    float* ss = m->ssm_st + ((size_t)j->slots[s] * m->nl + j->li) * ssm_len(m);
    float* y = m->y + s * di;
    const float* cv = m->conv_out + s * di;
    orc_ssm_d16(y + j0, ss + j0 * 16, dt + j0, cv + j0, L->a_log + j0 * 16, zp + dr, zp + dr + ds,
                L->d_vec + j0, (int)(j1 - j0));
    const float* z = m->xz + s * 2 * di + di;
    float* g = m->gated + s * di;
    size_t len = j1 - j0, body = len / 8 * 8;
    for (size_t i = 0; i < body; i++) g[j0 + i] = y[j0 + i] * (z[j0 + i] * lane_sigmoidf(z[j0 + i]));
    for (size_t i = body; i < len; i++) g[j0 + i] = y[j0 + i] * portable_silu(z[j0 + i]);
}

/* layer_norm_step (model.rs:193-200) / final_norm (model.rs:745-752). */
static void norm_into(float* out, const float* x, const float* w, const float* b, int d) {
    if (b) {
        orc_layer_norm(out, x, w, b, d, 1e-5f);
    } else {
        if (out != x) memcpy(out, x, sizeof(float) * d);
        orc_rms_norm(out, w, d, 1e-5f);
    }
}

/* forward_layers_normed_multi (model.rs:773-824) + compute_head_multi (model.rs:921-927):
 * bit-identical per stream to forward_into (model.rs:971-978), which the reference tests
 * (model.rs:1091-1134). */
int orc_mamba_forward(OrcMamba* m, uint32_t n, const uint32_t* slots, const uint32_t* tokens, float* out) {
    if (n == 0) return 0;
    if (n > m->cap || !slots || !tokens || !out) return 5;
    for (uint32_t b = 0; b < n; b++) {
        if (slots[b] >= m->cap || tokens[b] >= m->vocab) return 5;
        for (uint32_t c = 0; c < b; c++) if (slots[c] == slots[b]) return 5;
    }
    if (grow_scratch(m, n)) return 1;
    size_t d = m->d, di = m->di, xr = m->dr + 2 * m->ds;
    /* MambaState::maybe_periodic_reset (model.rs:315-320), before the embedding lookup. */
    for (uint32_t b = 0; b < n; b++) {
        uint32_t s = slots[b];
        if (m->reset_every > 0 && m->since[s] >= m->reset_every) reset_slot(m, s);
        m->since[s]++;
    }
    for (uint32_t b = 0; b < n; b++) mat_row(&m->emb, (int)tokens[b], m->x + b * d);
    for (uint32_t li = 0; li < m->nl; li++) {
        const Layer* L = &m->layers[li];
        for (uint32_t b = 0; b < n; b++) norm_into(m->normed + b * d, m->x + b * d, L->norm_w, L->norm_b, (int)d);
        gemv_multi(m, &L->in_proj, m->normed, d, m->xz, 2 * di, n);
        PhaseJob pj = { m, L, li, n, slots, (int)((di + 255) / 256) };
        pool_run((int)(n * pj.nblk), conv_block, &pj);
        gemv_multi(m, &L->x_proj, m->conv_out, di, m->zp, xr, n);
        pj.nblk = (int)((di + 63) / 64);
        pool_run((int)(n * pj.nblk), scan_block, &pj);
        gemv_multi(m, &L->out_proj, m->gated, di, m->res, d, n);
        for (uint32_t b = 0; b < n; b++)
            for (size_t k = 0; k < d; k++) m->x[b * d + k] += m->res[b * d + k];
    }
    for (uint32_t b = 0; b < n; b++) norm_into(m->x + b * d, m->x + b * d, m->norm_f_w, m->norm_f_b, (int)d);
    gemv_multi(m, m->head, m->x, d, out, m->vocab, n);
    return 0;
}

int orc_mamba_get_state(const OrcMamba* m, uint32_t slot, uint32_t layer, float* conv, float* ssm) {
    if (slot >= m->cap || layer >= m->nl) return 5;
    if (conv) memcpy(conv, m->conv_st + ((size_t)slot * m->nl + layer) * conv_len(m), sizeof(float) * conv_len(m));
    if (ssm) memcpy(ssm, m->ssm_st + ((size_t)slot * m->nl + layer) * ssm_len(m), sizeof(float) * ssm_len(m));
    return 0;
}

int orc_mamba_dequant(const OrcMamba* m, int which, uint32_t layer, float* out) {
    const Mat* w;
    if (which == 2) w = &m->emb;
    else if (layer >= m->nl) return 5;
    else if (which == 0) w = &m->layers[layer].in_proj;
    else if (which == 1) w = &m->layers[layer].out_proj;
    else if (which == 3) w = &m->layers[layer].x_proj;
    else if (which == 4) w = &m->layers[layer].dt_proj;
    else return 5;
    for (int r = 0; r < w->rows; r++) mat_row(w, r, out + (size_t)r * w->cols);
    return 0;
}
