// backend.hip — host side of libredukt_gpu.so: the plugin C ABI of redukt
// (src/domain/backend_ffi.rs, docs/api/PLUGIN-FFI-V2.md) over the gfx950 kernels.
//
// One process-global model, one non-blocking HIP stream at default priority, two
// disjoint state pools (v1: one slot; v2: the batch pool).  Weights are read from a
// .rbin file (F32) and, for the Q8 profiles, quantized here at load with the
// reference recipe before upload.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/redukt_backend.h"
#include "model.h"
#include "portable_math.h"

#pragma clang fp contract(off)

namespace rdk {

size_t TMat::bytes() const {
    if (!w) return 0;
    const size_t n = (size_t)rt * kRowTile * ks * kKStep;
    if (group == 0) return n * 4;
    return n + (size_t)rt * kRowTile * (group == cols ? 1 : ks / 2) * 4;
}

namespace {

constexpr uint32_t kRbinMagic = 0x55504752u;  // "RGPU"
constexpr uint32_t kFlagNormBias = 1u << 0;
constexpr uint32_t kFlagUntiedHead = 1u << 1;
constexpr int kMaxCols = 1024;  // d_model: activations of 32 streams staged in LDS, dt_rank in registers

enum ModelKind : uint32_t { kKindNone = 0, kKindMamba = 1, kKindRwkv = 2 };

struct Model {
    bool ready = false;
    uint32_t kind = kKindNone;
    Dims dims;                  // Mamba dims; for RWKV-7 only vocab, d and nl are set
    RDims rdims;                // RWKV-7
    std::vector<RLayer> rlayers;
    TMat r_emb, r_head;
    RowMat r_e_head;            // the RWKV-7 reference-order tier's head
    float* ln_out_w = nullptr;
    float* ln_out_b = nullptr;
    uint32_t profile = 0;
    std::vector<DLayer> layers;
    TMat emb, head_own;
    GMat g_emb, g_head_own;   // the wavefront-GEMV tier's embedding / untied head
    RowMat e_emb, e_head_own; // the reference-order tier's embedding / untied head
    bool gemv = false;        // weight profile bit 4
    bool exact = false;       // weight profile bit 6 or 7: the reference-order tier
    bool exact_fma = false;   // bit 7: its numeric contract 2 (fma-v1)
    bool r_a8 = false;        // weight profile bit 5: the RWKV-7 W8A8 tier
    bool r_exact = false;     // bit 6 on an RWKV-7 model: its F32 reference-order tier
    bool tied = true;
    float* norm_f_w = nullptr;
    float* norm_f_b = nullptr;
    std::vector<void*> allocs;
    unsigned char* arena = nullptr;   // current weight chunk and its fill
    size_t arena_used = 0;
    hipStream_t stream = nullptr;
    Pool v1, batch;
    StepRunner runner;
    uint32_t* d_err = nullptr;
    void* cdf_mem = nullptr;     // the device CDF's scratch (and CDF rows), grown on demand
    size_t cdf_bytes = 0;
    int device = 0;
    Probe probe;
};

Model G;

void log(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void log(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "[redukt-gpu-hip] ");
    vfprintf(stderr, fmt, ap);
    fprintf(stderr, "\n");
    va_end(ap);
}

// Weights go into 64 MB chunks in load order, 256-byte aligned, so that one layer's arrays
// sit together in a few large pages rather than in one small allocation each (fewer
// address-translation misses when a kernel first touches them).  An array larger than a
// quarter chunk gets its own allocation.  Every chunk ends in kArenaTail unused bytes, the
// slack a separate allocation would have had past its last array.
constexpr size_t kArenaChunk = (size_t)64 << 20;
constexpr size_t kArenaTail = (size_t)64 << 10;

void* arena_alloc(size_t bytes) {
    bytes = (bytes + 255) & ~(size_t)255;
    void* p = nullptr;
    if (bytes > kArenaChunk / 4) {
        if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
        G.allocs.push_back(p);
        return p;
    }
    if (G.arena == nullptr || G.arena_used + bytes > kArenaChunk) {
        if (hipMalloc(&p, kArenaChunk + kArenaTail) != hipSuccess) return nullptr;
        G.allocs.push_back(p);
        G.arena = (unsigned char*)p;
        G.arena_used = 0;
    }
    p = G.arena + G.arena_used;
    G.arena_used += bytes;
    return p;
}

template <typename T>
T* dev_upload(const T* host, size_t count) {
    T* p = (T*)arena_alloc(sizeof(T) * (count ? count : 1));
    if (p == nullptr) return nullptr;
    if (count && hipMemcpy(p, host, sizeof(T) * count, hipMemcpyHostToDevice) != hipSuccess) return nullptr;
    return p;
}

// Q8wMatrix::quantize (src/domain/gemv.rs:256-273): `group` columns per scale when it is
// a multiple of 8 dividing cols, else one scale per row; scale = max|w|/127 (1 for an
// all-zero group), q = clamp(round-half-away(w * (1/scale)), -127, 127).
int quantize(const float* w, int rows, int cols, int group, std::vector<int8_t>& q, std::vector<float>& sc) {
    if (!(group > 0 && group % 8 == 0 && cols % group == 0)) group = cols;
    const size_t total = (size_t)rows * cols, ng = total / group;
    q.resize(total);
    sc.resize(ng);
    for (size_t g = 0; g < ng; g++) {
        const float* wg = w + g * group;
        float amax = 0.0f;
        for (int i = 0; i < group; i++) amax = std::fmax(amax, std::fabs(wg[i]));
        const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / scale;
        for (int i = 0; i < group; i++) {
            float r = std::round(wg[i] * inv);
            r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
            q[g * group + i] = std::isnan(r) ? 0 : (int8_t)r;
        }
        sc[g] = scale;
    }
    return group;
}

// Tile a row-major [rows][cols] matrix for the matrix-core kernels (see TMat) and upload
// it, F32 or quantized.  quant_group: 0 = F32, else the requested Q8 group (cols = per
// row).
bool make_tmat(TMat& m, const float* w, int rows, int cols, int quant_group) {
    m.rows = rows;
    m.cols = cols;
    m.rt = (rows + kRowTile - 1) / kRowTile;
    const int kp = (cols + kKAlign - 1) / kKAlign * kKAlign;
    m.ks = kp / kKStep;
    const size_t elems = (size_t)m.rt * kRowTile * kp;
    auto f32_index = [&](int r, int k) {
        const int t = r / kRowTile, st = k / kKStep;
        const int lane = r % kRowTile + kRowTile * ((k % kKStep) / 8);
        return (((size_t)t * m.ks + st) * 64 + lane) * 8 + k % 8;
    };
    auto q8_index = [&](int r, int k) {
        const int t = r / kRowTile, st = k / kKStep;
        const int lane = r % kRowTile + kRowTile * ((k % kKStep) / 8);
        return ((((size_t)t * (m.ks / 2) + st / 2) * 64 + lane) * 2 + st % 2) * 8 + k % 8;
    };
    if (quant_group == 0) {
        std::vector<float> t(elems, 0.0f);
        for (int r = 0; r < rows; r++)
            for (int k = 0; k < cols; k++) t[f32_index(r, k)] = w[(size_t)r * cols + k];
        m.group = 0;
        m.w = dev_upload(t.data(), t.size());
        return m.w != nullptr;
    }
    std::vector<int8_t> q;
    std::vector<float> sc;
    m.group = quantize(w, rows, cols, quant_group, q, sc);
    std::vector<int8_t> t(elems, 0);
    for (int r = 0; r < rows; r++)
        for (int k = 0; k < cols; k++) t[q8_index(r, k)] = q[(size_t)r * cols + k];
    const int gpr = cols / m.group;               // scales per row as quantized
    const int spr = m.group == cols ? 1 : m.ks / 2;  // scales per row as stored
    std::vector<float> scp((size_t)m.rt * kRowTile * spr, 0.0f);
    for (int r = 0; r < rows; r++)
        for (int g = 0; g < gpr; g++) scp[(size_t)r * spr + g] = sc[(size_t)r * gpr + g];
    m.w = dev_upload(t.data(), t.size());
    m.scales = dev_upload(scp.data(), scp.size());
    return m.w && m.scales;
}

// Lay a row-major [rows][cols] f32 matrix out for the exact LoRA kernels (LMat:
// [cols / 8][rows8][8]) and upload it; cols must be a multiple of 8.
bool make_lmat(LMat& m, const float* w, int rows, int cols) {
    if (cols % 8 != 0) return false;
    m.rows = rows;
    m.cols = cols;
    m.rows8 = (rows + 7) / 8 * 8;
    std::vector<float> t((size_t)m.rows8 * cols, 0.0f);
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < cols; c++) t[((size_t)(c / 8) * m.rows8 + r) * 8 + c % 8] = w[(size_t)r * cols + c];
    m.w = dev_upload(t.data(), t.size());
    return m.w != nullptr;
}

// Lay a row-major [rows][cols] matrix out for the wavefront-GEMV kernels (see GMat) and
// upload it, F32 or quantized with one scale per row (the Q8 recipe with group = cols).
bool make_gmat(GMat& m, const float* w, int rows, int cols, bool q8) {
    int rpi = 0, cpl = 0;
    if (!gemv_shape(cols, rpi, cpl) || !gemv_cpl_supported(cpl)) return false;
    m.rows = rows;
    m.cols = cols;
    m.rpi = rpi;
    m.cpl = cpl;
    m.blocks = (rows + rpi - 1) / rpi;
    m.q8 = q8;
    const int per = 64 / rpi;
    const size_t n = (size_t)m.blocks * rpi * cols;
    std::vector<int8_t> q;
    std::vector<float> sc;
    if (q8) quantize(w, rows, cols, cols, q, sc);
    std::vector<int8_t> tq(q8 ? n : 0, 0);
    std::vector<float> tf(q8 ? 0 : n, 0.0f);
    for (int i = 0; i < m.blocks; i++)
        for (int j = 0; j < cpl; j++)
            for (int l = 0; l < 64; l++) {
                const int row = i * rpi + l % rpi, k0 = 16 * (l / rpi + per * j);
                if (row >= rows) continue;
                const size_t idx = (size_t)i * cpl + j;
                for (int e = 0; e < 16; e++) {
                    const size_t src = (size_t)row * cols + k0 + e;
                    if (q8)
                        tq[(idx * 64 + l) * 16 + e] = q[src];
                    else
                        tf[((idx * 4 + e / 4) * 64 + l) * 4 + e % 4] = w[src];
                }
            }
    if (q8) {
        std::vector<float> scp((size_t)m.blocks * rpi, 0.0f);
        for (int r = 0; r < rows; r++) scp[r] = sc[r];
        m.w = dev_upload(tq.data(), tq.size());
        m.scales = dev_upload(scp.data(), scp.size());
        return m.w && m.scales;
    }
    m.w = dev_upload(tf.data(), tf.size());
    return m.w != nullptr;
}

// Upload a row-major [rows][cols] matrix for the reference-order tier (RowMat): F32
// (quant_group 0) or the Q8 recipe with quant_group columns per scale (cols = per row),
// each row's 32-column blocks interleaved by column residue (column c of a block at
// 4 (c % 8) + c / 8).  Whole 32-column blocks only, in every row and every scale group.
bool make_rowmat(RowMat& m, const float* w, int rows, int cols, int quant_group) {
    m.rows = rows;
    m.cols = cols;
    if (cols % 32 != 0) return false;
    auto inter = [&](size_t r, int c) { return r * cols + (size_t)(c & ~31) + (size_t)(4 * (c & 7) + ((c & 31) >> 3)); };
    if (quant_group == 0) {
        m.group = 0;
        std::vector<float> t((size_t)rows * cols);
        for (int r = 0; r < rows; r++)
            for (int c = 0; c < cols; c++) t[inter(r, c)] = w[(size_t)r * cols + c];
        m.w = dev_upload(t.data(), t.size());
        return m.w != nullptr;
    }
    std::vector<int8_t> q;
    std::vector<float> sc;
    m.group = quantize(w, rows, cols, quant_group, q, sc);
    if (m.group % 32 != 0) return false;
    std::vector<int8_t> t((size_t)rows * cols);
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < cols; c++) t[inter(r, c)] = q[(size_t)r * cols + c];
    m.w = dev_upload(t.data(), t.size());
    m.scales = dev_upload(sc.data(), sc.size());
    return m.w && m.scales;
}

// The tile-shape fields of x_proj that size its outputs' row stride (xr_pad), for the tiers
// that keep x_proj in another layout.
void xproj_shape(TMat& t, int xr, int di) {
    t.rows = xr;
    t.cols = di;
    t.rt = (xr + kRowTile - 1) / kRowTile;
}

struct Reader {
    FILE* f;
    bool ok = true;
    std::vector<float> read(size_t count) {
        std::vector<float> v(count);
        if (ok && fread(v.data(), sizeof(float), count, f) != count) ok = false;
        return v;
    }
};

// .rbin v1/v2 (scripts/convert-weights-gpu.py:43-53, 152-197; reader semantics of
// plugins/redukt-gpu-cuda/mamba_cuda.cu:470-544).
int load_weights(const std::string& path, uint32_t profile) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) {
        log("cannot open: %s", path.c_str());
        return -1;
    }
    uint32_t h[11];
    Reader rd{f};
    bool hdr_ok = fread(h, 4, 11, f) == 11 && h[0] == kRbinMagic && (h[1] == 1 || h[1] == 2);
    if (hdr_ok) {
        hdr_ok = h[2] && h[3] && h[4] && h[5] && h[7] && h[8] && h[6] >= 2;
        if (h[1] == 2) hdr_ok = hdr_ok && h[10] <= 1 && !(h[10] == 0 && h[2] != 256);
        // Kernel limits: 16 SSM states per channel; d_model in whole 32-column k-steps and
        // at most kMaxCols; d_inner in whole 64-channel conv-branch blocks, at most 2048
        // (32 x_proj partials per row); x_proj rows (dt_rank <= 64) held in registers.
        hdr_ok = hdr_ok && h[5] == 16 && h[3] % 32 == 0 && h[4] % 64 == 0 && h[3] <= (uint32_t)kMaxCols &&
                 h[4] <= 2048 && h[7] <= 64;
    }
    if (!hdr_ok) {
        log("bad/unsupported .rbin header in %s", path.c_str());
        fclose(f);
        return -1;
    }
    Dims& D = G.dims;
    D.vocab = h[2]; D.d = h[3]; D.di = h[4]; D.ds = h[5]; D.dc = h[6]; D.dr = h[7]; D.nl = h[8]; D.flags = h[9];
    D.tokenizer = h[1] == 1 ? (D.vocab == 256 ? 0u : 1u) : h[10];
    const int quant = (profile & 3) == 0 ? 0 : ((profile & 3) == 1 ? 64 : (int)0x7fffffff);
    auto qgroup = [&](int cols) { return quant == 0 ? 0 : (quant == 0x7fffffff ? cols : quant); };
    const bool qsmall = quant != 0 && (profile & BACKEND_PROFILE_Q8_SMALL);
    const bool nb = D.flags & kFlagNormBias, uh = D.flags & kFlagUntiedHead;
    const bool gemv = (profile & BACKEND_PROFILE_GEMV) != 0;
    if (gemv) {
        // The GEMV tier: F32 or per-row int8, RMSNorm, a 4-wide conv, shapes it is compiled for.
        int r = 0, c = 0;
        const bool shapes = gemv_shape((int)D.d, r, c) && gemv_cpl_supported(c) && gemv_shape((int)D.di, r, c) &&
                            gemv_cpl_supported(c);
        if ((profile & 3) == 1 || nb || D.dc != 4 || !shapes) {
            log("the wavefront-GEMV tier needs F32 or per-row int8 weights, RMSNorm, d_conv 4 and compiled shapes");
            fclose(f);
            return -2;
        }
    }
    G.gemv = gemv;
    const bool exact = (profile & (BACKEND_PROFILE_EXACT | BACKEND_PROFILE_FMA)) != 0;
    G.exact = exact;
    G.exact_fma = (profile & BACKEND_PROFILE_FMA) != 0;
    const size_t V = D.vocab, d = D.d, di = D.di, dc = D.dc, dr = D.dr, xr = D.xr();
    log("rbin v%u: d=%u di=%u ds=%u dc=%u dr=%u nl=%u vs=%u flags=0x%02x tok=%u profile=%u", h[1], D.d, D.di, D.ds,
        D.dc, D.dr, D.nl, D.vocab, D.flags, D.tokenizer, profile);
    bool ok = true;
    {
        std::vector<float> e = rd.read(V * d);
        ok = rd.ok && (exact  ? make_rowmat(G.e_emb, e.data(), (int)V, (int)d, qgroup((int)d))
                       : gemv ? make_gmat(G.g_emb, e.data(), (int)V, (int)d, quant != 0)
                              : make_tmat(G.emb, e.data(), (int)V, (int)d, qgroup((int)d)));
    }
    G.layers.assign(D.nl, DLayer{});
    for (uint32_t i = 0; ok && i < D.nl; i++) {
        DLayer& L = G.layers[i];
        std::vector<float> t = rd.read(d);
        ok = rd.ok && (L.norm_w = dev_upload(t.data(), d));
        if (ok && nb) { t = rd.read(d); ok = rd.ok && (L.norm_b = dev_upload(t.data(), d)); }
        if (ok) {
            t = rd.read(2 * di * d);
            if (exact)
                ok = rd.ok && make_rowmat(L.e_in, t.data(), (int)(2 * di), (int)d, qgroup((int)d));
            else if (gemv)
                ok = rd.ok && make_gmat(L.g_in, t.data(), (int)(2 * di), (int)d, quant != 0);
            else
                ok = rd.ok && make_tmat(L.in_x, t.data(), (int)di, (int)d, qgroup((int)d)) &&
                     make_tmat(L.in_z, t.data() + di * d, (int)di, (int)d, qgroup((int)d));
        }
        if (ok) { t = rd.read(di * dc); ok = rd.ok && (L.conv_w = dev_upload(t.data(), di * dc)); }
        if (ok) { t = rd.read(di); ok = rd.ok && (L.conv_b = dev_upload(t.data(), di)); }
        if (ok) {
            t = rd.read(xr * di);
            if (exact) {
                xproj_shape(L.x_proj, (int)xr, (int)di);
                ok = rd.ok && make_rowmat(L.e_xp, t.data(), (int)xr, (int)di, qsmall ? qgroup((int)di) : 0);
            } else if (gemv) {
                // row-major for the GEMV tier's x_proj partials; the tile shape fields only
                xproj_shape(L.x_proj, (int)xr, (int)di);
                if (qsmall) {
                    std::vector<int8_t> q;
                    std::vector<float> sc;
                    quantize(t.data(), (int)xr, (int)di, (int)di, q, sc);
                    ok = rd.ok && (L.xp_q = dev_upload(q.data(), q.size())) && (L.xp_scales = dev_upload(sc.data(), sc.size()));
                } else {
                    ok = rd.ok && (L.xp_w = dev_upload(t.data(), t.size())) != nullptr;
                }
            } else {
                ok = rd.ok && make_tmat(L.x_proj, t.data(), (int)xr, (int)di, qsmall ? qgroup((int)di) : 0);
            }
        }
        if (ok) {
            t = rd.read(di * dr);
            ok = rd.ok;
            L.dt_pad = (int)((dr + 15) / 16 * 16);
            const size_t dp = (size_t)L.dt_pad;
            // Rows are stored in 16-byte chunks, chunk-major: chunk c of channel j at
            // [c][j], so the scan's 64 lanes read one contiguous kilobyte per chunk.
            if (ok && !qsmall) {
                std::vector<float> tp(di * dp, 0.0f);
                for (size_t j = 0; j < di; j++)
                    for (size_t k = 0; k < dr; k++) tp[((k / 4) * di + j) * 4 + k % 4] = t[j * dr + k];
                ok = (L.dt_w = dev_upload(tp.data(), tp.size())) != nullptr;
            } else if (ok) {
                std::vector<int8_t> q;
                std::vector<float> sc;
                // dt_rank <= 64: a 64-column group is the whole row or falls back to per-row.
                const int grp = quantize(t.data(), (int)di, (int)dr, qgroup((int)dr), q, sc);
                std::vector<int8_t> qp(di * dp, 0);
                for (size_t j = 0; j < di; j++)
                    for (size_t k = 0; k < dr; k++) qp[((k / 16) * di + j) * 16 + k % 16] = q[j * dr + k];
                ok = grp == (int)dr && (L.dt_q = dev_upload(qp.data(), qp.size())) &&
                     (L.dt_scales = dev_upload(sc.data(), sc.size()));
            }
        }
        if (ok) { t = rd.read(di); ok = rd.ok && (L.dt_b = dev_upload(t.data(), di)); }
        if (ok) {
            t = rd.read(di * 16);
            // exp(A_log) of every step (tensor.rs:1316), stored state-major [16][di]
            std::vector<float> ta(di * 16);
            for (size_t j = 0; j < di; j++)
                for (size_t n = 0; n < 16; n++) ta[n * di + j] = lane_exp_f(t[j * 16 + n]);
            ok = rd.ok && (L.a_exp = dev_upload(ta.data(), ta.size()));
        }
        if (ok) { t = rd.read(di); ok = rd.ok && (L.d_vec = dev_upload(t.data(), di)); }
        if (ok) {
            t = rd.read(d * di);
            ok = rd.ok && (exact  ? make_rowmat(L.e_out, t.data(), (int)d, (int)di, qgroup((int)di))
                           : gemv ? make_gmat(L.g_out, t.data(), (int)d, (int)di, quant != 0)
                                  : make_tmat(L.out_proj, t.data(), (int)d, (int)di, qgroup((int)di)));
        }
        if (ok && ((i + 1) % 8 == 0 || i + 1 == D.nl)) log("loaded layer %u/%u", i + 1, D.nl);
    }
    if (ok) { std::vector<float> t = rd.read(d); ok = rd.ok && (G.norm_f_w = dev_upload(t.data(), d)); }
    if (ok && nb) { std::vector<float> t = rd.read(d); ok = rd.ok && (G.norm_f_b = dev_upload(t.data(), d)); }
    G.tied = !uh;
    if (ok && uh) {
        std::vector<float> t = rd.read(V * d);
        ok = rd.ok && (exact  ? make_rowmat(G.e_head_own, t.data(), (int)V, (int)d, qgroup((int)d))
                       : gemv ? make_gmat(G.g_head_own, t.data(), (int)V, (int)d, quant != 0)
                              : make_tmat(G.head_own, t.data(), (int)V, (int)d, qgroup((int)d)));
    }
    fclose(f);
    return ok ? 0 : -1;
}

// RWKV-7 container (redukt_amd/rwkv.py): 16-word header (magic, version 3, model 2,
// vocab, d_model, n_head, head_size, n_layer, d_ffn, four LoRA ranks, flags, tokenizer,
// 0), then the f32 tensors in that module's order.  Quantized profiles apply the Q8
// recipe to receptance, key, value, output, FFN key/value and the head; the embedding
// and the LoRAs stay F32 (src/infrastructure/rwkv7/model.rs:997-1059).
int load_rwkv(const std::string& path, uint32_t profile) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) {
        log("cannot open: %s", path.c_str());
        return -1;
    }
    uint32_t h[16];
    Reader rd{f};
    bool hdr_ok = fread(h, 4, 16, f) == 16 && h[0] == kRbinMagic && h[1] == 3 && h[2] == 2;
    // Kernel limits: 64-wide heads; d_model in whole 64-column k-pairs, at most 1024.
    hdr_ok = hdr_ok && h[3] && h[4] == h[5] * h[6] && h[6] == 64 && h[4] % 64 == 0 && h[4] <= 1024 && h[7] &&
             h[8] && h[8] % 16 == 0 && h[9] && h[10] && h[11] && h[12] && h[9] <= 512 && h[10] <= 512 &&
             h[11] <= 512 && h[12] <= 512 && h[14] <= 1;
    if (!hdr_ok) {
        log("bad/unsupported RWKV-7 header in %s", path.c_str());
        fclose(f);
        return -1;
    }
    RDims& R = G.rdims;
    R.vocab = h[3]; R.d = h[4]; R.h = h[5]; R.n = h[6]; R.nl = h[7]; R.f = h[8];
    R.lora[kLoraW] = h[9]; R.lora[kLoraA] = h[10]; R.lora[kLoraV] = h[11]; R.lora[kLoraG] = h[12];
    R.g1k = h[13] & 1u;
    G.dims = Dims{};
    G.dims.vocab = R.vocab;
    G.dims.d = R.d;
    G.dims.nl = R.nl;
    G.dims.tokenizer = h[14];
    G.r_a8 = (profile & BACKEND_PROFILE_W8A8) != 0;
    G.r_exact = (profile & BACKEND_PROFILE_EXACT) != 0;
    if ((G.r_a8 || G.r_exact) && (R.lora[0] % 8 || R.lora[1] % 8 || R.lora[2] % 8 || R.lora[3] % 8)) {
        log("the W8A8 and reference-order tiers need LoRA ranks in multiples of 8");
        fclose(f);
        return -2;
    }
    // the reference-order projections stage four streams' input rows in LDS (64 KB at most)
    if (G.r_exact && (R.f % 32 != 0 || R.f > 4096)) {
        log("the reference-order tier needs d_ffn in whole 32-column blocks, at most 4096");
        fclose(f);
        return -2;
    }
    const int quant = (profile & 3) == 0 ? 0 : ((profile & 3) == 1 ? 64 : (int)0x7fffffff);
    auto qgroup = [&](int cols) { return quant == 0 ? 0 : (quant == 0x7fffffff ? cols : quant); };
    const size_t V = R.vocab, d = R.d, ff = R.f;
    log("rwkv7: d=%u heads=%u x %u layers=%u d_ffn=%u lora=%u/%u/%u/%u vocab=%u g1k=%u profile=%u", R.d, R.h, R.n,
        R.nl, R.f, R.lora[kLoraW], R.lora[kLoraA], R.lora[kLoraV], R.lora[kLoraG], R.vocab, R.g1k, profile);
    bool ok = true;
    auto vec = [&](float*& dst) {
        std::vector<float> t = rd.read(d);
        ok = ok && rd.ok && (dst = dev_upload(t.data(), d)) != nullptr;
    };
    auto mat = [&](TMat& m, size_t rows, size_t cols, int group) {
        std::vector<float> t = rd.read(rows * cols);
        ok = ok && rd.ok && make_tmat(m, t.data(), (int)rows, (int)cols, group);
    };
    // A projection: tiled for the matrix cores, or F32 rows for the reference-order tier.
    auto proj = [&](TMat& m, RowMat& e, size_t rows, size_t cols) {
        if (!G.r_exact) {
            mat(m, rows, cols, qgroup((int)cols));
            return;
        }
        std::vector<float> t = rd.read(rows * cols);
        ok = ok && rd.ok && make_rowmat(e, t.data(), (int)rows, (int)cols, 0);
    };
    // A LoRA stage: tiled for the matrix cores, or laid out for the exact kernels of the
    // W8A8 and reference-order tiers.
    auto lora = [&](RLayer& L, int k, bool first, size_t rows, size_t cols) {
        std::vector<float> t = rd.read(rows * cols);
        if (G.r_a8 || G.r_exact)
            ok = ok && rd.ok && make_lmat(first ? L.x1[k] : L.x2[k], t.data(), (int)rows, (int)cols);
        else ok = ok && rd.ok && make_tmat(first ? L.l1[k] : L.l2[k], t.data(), (int)rows, (int)cols, 0);
    };
    mat(G.r_emb, V, d, 0);
    G.rlayers.assign(R.nl, RLayer{});
    for (uint32_t i = 0; ok && i < R.nl; i++) {
        RLayer& L = G.rlayers[i];
        vec(L.ln1_w); vec(L.ln1_b); vec(L.ln2_w); vec(L.ln2_b);
        for (int k = 0; k < 6; k++) vec(L.mix[k]);
        vec(L.w0);
        lora(L, kLoraW, true, R.lora[kLoraW], d);
        lora(L, kLoraW, false, d, R.lora[kLoraW]);
        vec(L.a0);
        lora(L, kLoraA, true, R.lora[kLoraA], d);
        lora(L, kLoraA, false, d, R.lora[kLoraA]);
        vec(L.v0);
        lora(L, kLoraV, true, R.lora[kLoraV], d);
        lora(L, kLoraV, false, d, R.lora[kLoraV]);
        lora(L, kLoraG, true, R.lora[kLoraG], d);
        lora(L, kLoraG, false, d, R.lora[kLoraG]);
        vec(L.k_k); vec(L.k_a); vec(L.r_k);
        proj(L.r, L.e_r, d, d);
        proj(L.k, L.e_k, d, d);
        proj(L.v, L.e_v, d, d);
        proj(L.o, L.e_o, d, d);
        vec(L.ln_x_w); vec(L.ln_x_b); vec(L.ffn_x_k);
        proj(L.fk, L.e_fk, ff, d);
        proj(L.fv, L.e_fv, d, ff);
        if (ok && ((i + 1) % 4 == 0 || i + 1 == R.nl)) log("loaded layer %u/%u", i + 1, R.nl);
    }
    vec(G.ln_out_w);
    vec(G.ln_out_b);
    proj(G.r_head, G.r_e_head, V, d);
    if (ok) {
        char extra;
        ok = fread(&extra, 1, 1, f) == 0;
    }
    fclose(f);
    return ok ? 0 : -1;
}

// Model kind from the first header words: "RGPU" version 3 model 2 is RWKV-7, anything
// else goes to the .rbin (Mamba) reader.
uint32_t file_kind(const std::string& path) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return kKindMamba;
    uint32_t h[3] = {0, 0, 0};
    const bool got = fread(h, 4, 3, f) == 3;
    fclose(f);
    return got && h[0] == kRbinMagic && h[1] == 3 && h[2] == 2 ? kKindRwkv : kKindMamba;
}

void dev_free_all() {
    for (void* p : G.allocs) (void)hipFree(p);
    G.allocs.clear();
    G.arena = nullptr;
    G.arena_used = 0;
}

// Outputs reach host memory in rounds of up to kOutRoundBytes through a pinned buffer:
// every chunk of a round is copied D2H at once, each with its own event, and all the host
// threads of copy_pool() move each chunk into the caller's buffer, a slice each, as soon as
// its DMA ends, while the next chunk's DMA runs.  Each D2H copy costs about 8 us on top of
// its bytes (53 GB/s pinned; 6.4 MB: one copy 120 us, seven 1 MB copies 175 us), so a round
// is cut into 2 to kOutMaxChunks chunks of about kOutChunkTarget bytes.  Measured on
// Mamba-130M int8 (tok/s through forward_batch, 32 / 128 streams): one thread per chunk,
// two chunks 47.6K / 77.5K; eight threads slicing every chunk, two chunks 55.2K / 97.5K,
// four chunks 53.0K / 101.2K.
constexpr size_t kOutChunkTarget = (size_t)4 << 20;
constexpr size_t kOutMaxChunks = 4;
constexpr size_t kOutRoundBytes = (size_t)32 << 20;
constexpr unsigned kCopyThreadsMax = 8;   // the caller's thread and at most seven helpers

bool out_stage_alloc(Pool& p, size_t out_bytes) {
    // at least 4 u32 a stream: the CDF readers' results come back through it in one piece
    p.out_stage_bytes = std::max(std::min(kOutRoundBytes, (out_bytes + 255) & ~(size_t)255),
                                 ((size_t)p.cap * 16 + 255) & ~(size_t)255);
    if (hipHostMalloc((void**)&p.h_out, p.out_stage_bytes, hipHostMallocDefault) != hipSuccess) {
        p.h_out = nullptr;
        return false;
    }
    static_assert(kOutMaxChunks <= sizeof(Pool::out_ev) / sizeof(hipEvent_t), "events per round");
    for (size_t c = 0; c < kOutMaxChunks; c++)
        if (hipEventCreateWithFlags(&p.out_ev[c], hipEventDisableTiming) != hipSuccess) return false;
    return true;
}

// The host side of the queued calls' buffers (the device inputs are carved with the pool).
bool queued_alloc(Pool& p, size_t n) {
    for (Pool::Queued& q : p.queued) {
        if (hipHostMalloc((void**)&q.h_in, sizeof(uint32_t) * 3 * n, hipHostMallocDefault) != hipSuccess) {
            q.h_in = nullptr;
            return false;
        }
        if (hipHostMalloc((void**)&q.h_res, sizeof(uint32_t) * 3 * n, hipHostMallocDefault) != hipSuccess) {
            q.h_res = nullptr;
            return false;
        }
        if (hipEventCreateWithFlags(&q.done, hipEventDisableTiming) != hipSuccess) {
            q.done = nullptr;
            return false;
        }
    }
    return true;
}

// Host threads that copy a round's chunks: one job per round, body(t) run once by each of
// the threads() threads (t = 0 is the caller).  A job ends when every helper has finished
// its part, so nothing of a job is touched after run() returns.  The helpers start on first
// use: REDUKT_HOST_THREADS of them counting the caller (else the CPU count), at most
// kCopyThreadsMax; a helper that cannot be started (a thread limit) leaves the job to the
// threads that did start, down to the caller alone, so no exception leaves the library.
class CopyPool {
public:
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> g(mu_);
            stop_ = true;
            ++gen_;
        }
        cv_.notify_all();
        for (auto& t : th_) t.join();
    }
    unsigned threads() {
        if (!started_) start();
        return 1u + (unsigned)th_.size();
    }
    // body(t) on each thread t in [0, threads()); false if any failed.
    bool run(const std::function<bool(unsigned)>& body) {
        const unsigned nt = threads();
        if (nt == 1) return body(0);
        {
            std::lock_guard<std::mutex> g(mu_);
            body_ = &body;
            busy_ = nt - 1;
            ok_ = true;
            ++gen_;
        }
        cv_.notify_all();
        const bool ok = body(0);
        std::unique_lock<std::mutex> g(mu_);
        done_.wait(g, [&] { return busy_ == 0; });
        body_ = nullptr;
        return ok && ok_;
    }

private:
    void start() {
        started_ = true;
        unsigned want = std::thread::hardware_concurrency();
        if (const char* e = getenv("REDUKT_HOST_THREADS"))
            if (*e) want = (unsigned)strtoul(e, nullptr, 10);
        want = std::max(1u, std::min(want, kCopyThreadsMax));
        try {
            th_.reserve(want - 1);
            for (unsigned i = 1; i < want; i++) th_.emplace_back([this, i] { loop(i); });
        } catch (...) {
            // run with the helpers that started
        }
    }
    void loop(unsigned id) {
        uint64_t seen = 0;
        for (;;) {
            const std::function<bool(unsigned)>* body;
            {
                std::unique_lock<std::mutex> g(mu_);
                cv_.wait(g, [&] { return gen_ != seen; });
                seen = gen_;
                if (stop_) return;
                body = body_;
            }
            const bool ok = (*body)(id);
            std::lock_guard<std::mutex> g(mu_);
            ok_ = ok_ && ok;
            if (--busy_ == 0) done_.notify_all();
        }
    }
    std::vector<std::thread> th_;
    std::mutex mu_;
    std::condition_variable cv_, done_;
    uint64_t gen_ = 0;
    bool stop_ = false, ok_ = true, started_ = false;
    unsigned busy_ = 0;
    const std::function<bool(unsigned)>* body_ = nullptr;
};

CopyPool& copy_pool() {
    static CopyPool pool;
    return pool;
}

void pool_free(Pool& p) {
    if (p.block) (void)hipFree(p.block);
    if (p.h_slots) (void)hipHostFree(p.h_slots);
    if (p.h_out) (void)hipHostFree(p.h_out);
    for (hipEvent_t& e : p.out_ev)
        if (e) (void)hipEventDestroy(e);
    for (Pool::Queued& q : p.queued) {
        if (q.h_in) (void)hipHostFree(q.h_in);
        if (q.h_res) (void)hipHostFree(q.h_res);
        if (q.done) (void)hipEventDestroy(q.done);
    }
    free(p.seen);
    p = Pool{};
}

// A pool's device arrays are carved from one zeroed allocation (256-byte aligned, in the
// order given: the per-step scratch first, the recurrent state last), so a step touches
// few, large pages.  The layout function runs twice: to size the block, then to carve it.
struct Carve {
    unsigned char* base = nullptr;
    size_t off = 0;
    template <typename T>
    void take(T*& p, size_t count) {
        off = (off + 255) & ~(size_t)255;
        p = base ? (T*)(base + off) : nullptr;
        off += sizeof(T) * (count ? count : 1);
    }
};

template <typename F>
bool pool_carve(Pool& p, F&& layout) {
    Carve c;
    layout(c);
    const size_t bytes = c.off + kArenaTail;
    if (hipMalloc(&p.block, bytes) != hipSuccess) {
        p.block = nullptr;
        return false;
    }
    if (hipMemset(p.block, 0, bytes) != hipSuccess) return false;
    c.base = (unsigned char*)p.block;
    c.off = 0;
    layout(c);
    return true;
}

uint32_t vocab_of_model() { return G.dims.vocab; }

size_t slot_words(uint32_t cap) { return ((size_t)cap + kSlotWordAlign - 1) / kSlotWordAlign * kSlotWordAlign; }

bool pool_alloc_rwkv(Pool& p, uint32_t cap) {
    const RDims& R = G.rdims;
    const size_t n = cap, d = R.d;
    const RwkvSizes z = rwkv_sizes(R, cap, G.r_a8 || G.r_exact, G.r_exact);
    p = Pool{};
    p.cap = cap;
    p.scap = cap + 1;
    p.xcap = cap;
    p.gcap = (cap + 15) / 16;
    bool ok = pool_carve(p, [&](Carve& c) {
        c.take(p.slots, slot_words(cap));
        c.take(p.d_slots, 3 * n);  // a step's n slots, its n tokens, then a word per stream for the CDF readers (one H2D copy)
        for (Pool::Queued& q : p.queued) c.take(q.d_in, 3 * n);
        c.take(p.x, n * d);
        c.take(p.vfirst, n * d);
        c.take(p.rkv, n * 3 * d);
        c.take(p.lorad, n * 4 * d);
        c.take(p.mixl, 6 * z.mixl);
        c.take(p.loral, z.loral);
        c.take(p.gatedl, z.gatedl);
        c.take(p.ffnl, z.mixl);
        c.take(p.actl, z.actl);
        c.take(p.headl, z.mixl);
        c.take(p.mixf, z.mixf);
        c.take(p.lorah, z.lorah);
        c.take(p.aq, z.aq);
        c.take(p.as, z.as);
        c.take(p.gatedf, z.gatedf);
        c.take(p.actf, z.actf);
        c.take(p.pmax, z.pmax);
        c.take(p.out, n * R.vocab);
        c.take(p.x_att, z.state_d);
        c.take(p.x_ffn, z.state_d);
        c.take(p.wkv, z.wkv);
    });
    ok = ok && hipHostMalloc((void**)&p.h_slots, sizeof(uint32_t) * 3 * n, hipHostMallocDefault) == hipSuccess;
    ok = ok && queued_alloc(p, n);

    ok = ok && (p.seen = (uint8_t*)calloc(n, 1)) != nullptr;
    ok = ok && out_stage_alloc(p, (size_t)n * vocab_of_model() * sizeof(float));
    return ok;
}

bool pool_alloc(Pool& p, uint32_t cap) {
    if (G.kind == kKindRwkv) return pool_alloc_rwkv(p, cap);
    const Dims& D = G.dims;
    const size_t n = cap, d = D.d, di = D.di;
    p = Pool{};
    p.cap = cap;
    p.scap = cap + 1;
    p.xcap = cap;
    p.gcap = (cap + 15) / 16;
    const size_t ns = p.scap;
    bool ok = pool_carve(p, [&](Carve& c) {
        c.take(p.slots, slot_words(cap));
        c.take(p.d_slots, 3 * n);  // a step's n slots, its n tokens, then a word per stream for the CDF readers (one H2D copy)
        for (Pool::Queued& q : p.queued) c.take(q.d_in, 3 * n);
        c.take(p.x, n * d);
        c.take(p.xw, xw_elems(D, cap));
        c.take(p.ssp, ssp_floats(D, cap));
        c.take(p.u, n * di);
        c.take(p.z, n * di);
        c.take(p.xpart, xpart_floats(D, cap));
        c.take(p.glimb, glimb_elems(D, cap));
        c.take(p.g32, G.gemv || G.exact ? n * di : 0);
        c.take(p.normed, G.exact ? n * d : 0);
        c.take(p.out, n * D.vocab);
        c.take(p.conv, (size_t)D.nl * ns * di * (D.dc - 1));
        c.take(p.ssm, (size_t)D.nl * ns * di * 16);
    });
    ok = ok && hipHostMalloc((void**)&p.h_slots, sizeof(uint32_t) * 3 * n, hipHostMallocDefault) == hipSuccess;
    ok = ok && queued_alloc(p, n);

    ok = ok && (p.seen = (uint8_t*)calloc(n, 1)) != nullptr;
    ok = ok && out_stage_alloc(p, (size_t)n * vocab_of_model() * sizeof(float));
    return ok;
}

void free_model() {
    if (G.stream) (void)hipStreamSynchronize(G.stream);
    G.runner.release();
    pool_free(G.v1);
    pool_free(G.batch);
    if (G.cdf_mem) (void)hipFree(G.cdf_mem);
    dev_free_all();
    if (G.stream) (void)hipStreamDestroy(G.stream);
    G = Model{};
}

ModelView model_view() {
    return ModelView{&G.dims, G.layers.data(), &G.emb, G.tied ? &G.emb : &G.head_own, G.norm_f_w, G.norm_f_b,
                     (G.profile & BACKEND_PROFILE_EXACT_SCAN) != 0};
}

ExactView exact_view() {
    return ExactView{&G.dims, G.layers.data(), &G.e_emb, G.tied ? &G.e_emb : &G.e_head_own, G.norm_f_w, G.norm_f_b,
                     G.exact_fma};
}

GemvView gemv_view() {
    return GemvView{&G.dims, G.layers.data(), &G.g_emb, G.tied ? &G.g_emb : &G.g_head_own, G.norm_f_w,
                    (G.profile & BACKEND_PROFILE_EXACT_SCAN) != 0};
}

hipError_t run_step(Pool& p, uint32_t n, const uint32_t* slots, const uint32_t* tokens, float* out, bool probs,
                    bool check) {
    StepIO io{n, slots, tokens, out, probs, check, G.d_err};
    if (G.kind == kKindRwkv) {
        const RwkvStep src(RwkvView{&G.rdims, G.rlayers.data(), &G.r_emb, &G.r_head, G.ln_out_w, G.ln_out_b, G.r_a8,
                                    G.r_exact, &G.r_e_head});
        return G.runner.run(src, p, io, G.stream, &G.probe);
    }
    if (G.gemv) {
        const GemvStep src(gemv_view());
        return G.runner.run(src, p, io, G.stream, &G.probe);
    }
    if (G.exact) {
        const ExactStep src(exact_view());
        return G.runner.run(src, p, io, G.stream, &G.probe);
    }
    const MambaStep src(model_view());
    return G.runner.run(src, p, io, G.stream, &G.probe);
}

// Wait for an event by polling it: the copy threads pick a chunk up within a microsecond of
// its DMA's end (a blocking wait can sleep for tens of microseconds).
bool event_wait(hipEvent_t e) {
    for (;;) {
        const hipError_t r = hipEventQuery(e);
        if (r == hipSuccess) return true;
        if (r != hipErrorNotReady) return false;
        std::this_thread::yield();
    }
}

// The first `bytes` of the device array src into the caller's host buffer dst, through the
// pool's pinned staging, a round at a time: all of a round's chunks are queued D2H (each
// followed by its event) behind the step; the caller alone polls for the first chunk (which
// lands only after the whole step), then every copy thread walks the chunks in order, waits
// for each one's event and moves its slice of the chunk into dst, while the later chunks
// are still in flight.  Returns when every byte is in dst.
bool copy_out(Pool& p, void* dst, const void* src, size_t bytes) {
    for (size_t r0 = 0; r0 < bytes; r0 += p.out_stage_bytes) {
        const size_t rb = std::min(p.out_stage_bytes, bytes - r0);
        const size_t want = std::min(kOutMaxChunks, std::max<size_t>(2, (rb + kOutChunkTarget - 1) / kOutChunkTarget));
        const size_t cb = ((rb + want - 1) / want + 255) & ~(size_t)255;
        const size_t chunks = (rb + cb - 1) / cb;
        for (size_t c = 0; c < chunks; c++) {
            const size_t off = c * cb, len = std::min(cb, rb - off);
            if (hipMemcpyAsync(p.h_out + off, (const unsigned char*)src + r0 + off, len, hipMemcpyDeviceToHost,
                               G.stream) != hipSuccess ||
                hipEventRecord(p.out_ev[c], G.stream) != hipSuccess)
                return false;
        }
        if (!event_wait(p.out_ev[0])) return false;
        const unsigned nt = copy_pool().threads();
        const bool ok = copy_pool().run([&](unsigned t) {
            for (size_t c = 0; c < chunks; c++) {
                if (c > 0 && !event_wait(p.out_ev[c])) return false;
                const size_t off = c * cb, len = std::min(cb, rb - off);
                // slice t of the chunk, 64-byte aligned
                const size_t per = ((len + nt - 1) / nt + 63) & ~(size_t)63;
                const size_t s0 = std::min(len, (size_t)t * per), s1 = std::min(len, s0 + per);
                if (s1 > s0) memcpy((unsigned char*)dst + r0 + off + s0, p.h_out + off + s0, s1 - s0);
            }
            return true;
        });
        if (!ok) return false;
    }
    return true;
}

// pool_forward semantics (mamba_cuda.cu:604-635): validate on the host (nothing is
// launched on INVALID_ARGUMENT), stage slots/tokens through pinned memory, enqueue the
// step, copy the n rows back to the caller (through pinned staging, chunked) and wait.
int pool_forward(Pool& p, uint32_t n, const uint32_t* slots, const uint32_t* tokens, float* out, bool probs) {
    memset(p.seen, 0, p.cap);
    for (uint32_t b = 0; b < n; b++) {
        if (slots[b] >= p.cap || p.seen[slots[b]] || tokens[b] >= G.dims.vocab) return BACKEND_INVALID_ARGUMENT;
        p.seen[slots[b]] = 1;
    }
    // the n slots, then the n tokens, in one staging run and one copy
    memcpy(p.h_slots, slots, sizeof(uint32_t) * n);
    memcpy(p.h_slots + n, tokens, sizeof(uint32_t) * n);
    if (hipMemcpyAsync(p.d_slots, p.h_slots, sizeof(uint32_t) * 2 * n, hipMemcpyHostToDevice, G.stream) != hipSuccess)
        return BACKEND_FORWARD_FAILED;
    if (run_step(p, n, p.d_slots, p.d_slots + n, p.out, probs, false) != hipSuccess) return BACKEND_FORWARD_FAILED;
    if (!copy_out(p, out, p.out, sizeof(float) * n * G.dims.vocab)) return BACKEND_FORWARD_FAILED;
    return BACKEND_OK;
}

// pool_reset semantics (mamba_cuda.cu:637-658), validated before anything is queued.
int pool_reset(Pool& p, uint32_t n, const uint32_t* slots) {
    for (uint32_t b = 0; b < n; b++) {
        const uint32_t s = slots ? slots[b] : b;
        if (s >= p.cap) return BACKEND_INVALID_ARGUMENT;
    }
    if (n == 0) return BACKEND_OK;
    // Every earlier call that used p.h_slots ended with a stream synchronize, so the
    // staging buffer is free to overwrite.
    for (uint32_t b = 0; b < n; b++) p.h_slots[b] = slots ? slots[b] : b;
    if (hipMemcpyAsync(p.d_slots, p.h_slots, sizeof(uint32_t) * n, hipMemcpyHostToDevice, G.stream) != hipSuccess)
        return BACKEND_FORWARD_FAILED;
    const hipError_t e = G.kind == kKindRwkv ? enqueue_reset_rwkv(G.rdims, p, p.d_slots, n, G.stream)
                                             : enqueue_reset(G.dims, p, p.d_slots, n, G.stream);
    if (e != hipSuccess) return BACKEND_FORWARD_FAILED;
    if (hipStreamSynchronize(G.stream) != hipSuccess) return BACKEND_FORWARD_FAILED;
    return BACKEND_OK;
}

std::string rbin_path(const uint8_t* weights_path) {
    std::string p((const char*)weights_path);
    if (p.size() < 5 || p.compare(p.size() - 5, 5, ".rbin") != 0) p += "/model.rbin";
    return p;
}

uint32_t env_weight_profile() {
    const char* e = getenv("REDUKT_GPU_PROFILE");
    if (!e || !*e || !strcmp(e, "f32")) return BACKEND_PROFILE_F32;
    if (!strcmp(e, "q8")) return BACKEND_PROFILE_Q8_G64;
    if (!strcmp(e, "q8row")) return BACKEND_PROFILE_Q8_ROW;
    if (!strcmp(e, "q8row-all")) return BACKEND_PROFILE_Q8_ROW | BACKEND_PROFILE_Q8_SMALL;
    if (!strcmp(e, "q8-all")) return BACKEND_PROFILE_Q8_G64 | BACKEND_PROFILE_Q8_SMALL;
    // the bit-exact tiers under the reference's own profile names and numeric contracts
    if (!strcmp(e, "f32-ref")) return BACKEND_PROFILE_F32 | BACKEND_PROFILE_EXACT;
    if (!strcmp(e, "q8-ref")) return BACKEND_PROFILE_Q8_G64 | BACKEND_PROFILE_EXACT;
    if (!strcmp(e, "f32-ref-fma")) return BACKEND_PROFILE_F32 | BACKEND_PROFILE_EXACT | BACKEND_PROFILE_FMA;
    if (!strcmp(e, "q8-ref-fma")) return BACKEND_PROFILE_Q8_G64 | BACKEND_PROFILE_EXACT | BACKEND_PROFILE_FMA;
    if (!strcmp(e, "q8row-w8a8")) return BACKEND_PROFILE_Q8_ROW | BACKEND_PROFILE_W8A8;
    return (uint32_t)strtoul(e, nullptr, 0) & 255u;
}

// REDUKT_GPU_SPLIT: most parts (sub-batches on their own streams) a step is split into.
uint32_t env_split() {
    const char* e = getenv("REDUKT_GPU_SPLIT");
    if (!e || !*e) return kDefaultSplit;
    return (uint32_t)strtoul(e, nullptr, 10);
}

// REDUKT_GPU_FLOW: smallest step (streams) that runs the persistent step kernel; 0 never.
uint32_t env_flow_from() {
    const char* e = getenv("REDUKT_GPU_FLOW");
    if (!e || !*e) return kDefaultFlowFrom;
    return (uint32_t)strtoul(e, nullptr, 10);
}

// REDUKT_GPU_SKEW: launches of part 0 ahead of the other parts of a split step.
uint32_t env_skew() {
    const char* e = getenv("REDUKT_GPU_SKEW");
    if (!e || !*e) return kDefaultSkew;
    return (uint32_t)strtoul(e, nullptr, 10);
}

// REDUKT_GPU_PART_MIN: fewest streams per part.
uint32_t env_part_min() {
    const char* e = getenv("REDUKT_GPU_PART_MIN");
    if (!e || !*e) return kMinPartStreams;
    return (uint32_t)strtoul(e, nullptr, 10);
}

uint32_t env_profile() {
    const char* x = getenv("REDUKT_GPU_EXACT_SCAN");
    return env_weight_profile() | (x && *x && strcmp(x, "0") ? BACKEND_PROFILE_EXACT_SCAN : 0u);
}

// ---------------------------------------------------------------- allocation-free step
// The per-step scratch of redukt_backend_forward_batch_device_noalloc (activations, limbs,
// x_proj partials, the validated slot list) lives in this file-scope device array, one
// copy per device the library runs on, held until the process ends.  Host code uses only
// the address hipGetSymbolAddress returns for the current device (noalloc_base), never the
// array's name.  Every call clears the part it carves before the step, and every call on a
// device shares it: calls that overlap on one device race (calls on the library's stream
// are ordered, so only calls from several threads can overlap).
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
void* g_noalloc_base[kMaxDevices] = {};

// Once per device, with that device current (the library's init).
bool noalloc_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return false;
    if (g_noalloc_base[device]) return true;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
        log("no-alloc scratch: hipGetSymbolAddress failed (%s)", hipGetErrorString(e));
        return false;
    }
    g_noalloc_base[device] = ptr;
    return true;
}

// The batch pool's state with the per-step scratch of n streams carved from the device's
// scratch array (the x_proj partials with row stride n); false if it does not fit.
bool noalloc_view(Pool& v, uint32_t n, unsigned char* base, size_t* used) {
    const Dims& D = G.dims;
    v = G.batch;
    v.xcap = n;
    v.gcap = (n + 15) / 16;
    Carve c;
    c.base = base;
    c.take(v.slots, slot_words(n));
    c.take(v.x, (size_t)n * D.d);
    c.take(v.xw, xw_elems(D, n));
    c.take(v.ssp, ssp_floats(D, n));
    c.take(v.u, (size_t)n * D.di);
    c.take(v.z, (size_t)n * D.di);
    c.take(v.xpart, xpart_floats(D, n));
    c.take(v.glimb, glimb_elems(D, n));
    if (G.gemv || G.exact) c.take(v.g32, (size_t)n * D.di);
    if (G.exact) c.take(v.normed, (size_t)n * D.d);
    *used = (c.off + 255) & ~(size_t)255;
    v.out = nullptr;
    v.d_slots = v.h_slots = nullptr;
    v.seen = nullptr;
    return *used <= kNoAllocScratchBytes;
}

__global__ __launch_bounds__(256) void k_clear(uint4* p, size_t n16) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

int init_common(const uint8_t* weights_path, int32_t device_id, uint32_t profile, BackendInfo* info_out) {
    if (!weights_path || !info_out) return BACKEND_INIT_FAILED;
    if (G.ready || G.stream) free_model();
    if ((profile & 3) == 3) return BACKEND_INIT_FAILED;
    const std::string path = rbin_path(weights_path);
    log("init: weights=%s device=%d profile=%u", path.c_str(), device_id, profile);
    G.device = device_id >= 0 ? device_id : 0;
    if (hipSetDevice(G.device) != hipSuccess ||
        hipStreamCreateWithFlags(&G.stream, hipStreamNonBlocking) != hipSuccess) {
        free_model();
        return BACKEND_INIT_FAILED;
    }
    (void)noalloc_setup(G.device);  // a failure only disables the allocation-free entry point
    G.profile = profile;
    G.runner.set_split(env_split(), env_part_min());
    G.runner.set_flow(env_flow_from());
    G.runner.set_skew(env_skew());
    G.kind = file_kind(path);
    if (G.kind == kKindRwkv && (profile & BACKEND_PROFILE_GEMV)) {
        log("the wavefront-GEMV tier serves Mamba models only");
        free_model();
        return BACKEND_INIT_FAILED;
    }
    if ((profile & (BACKEND_PROFILE_EXACT | BACKEND_PROFILE_FMA)) && G.kind == kKindMamba &&
        (profile & (BACKEND_PROFILE_GEMV | BACKEND_PROFILE_W8A8))) {
        log("the reference-order tier is a tier of its own, apart from the GEMV and W8A8 tiers");
        free_model();
        return BACKEND_INIT_FAILED;
    }
    // RWKV-7 in the reference's arithmetic: F32 in numeric contract 1 here (the reference's
    // RWKV-7 GEMVs have no fma-v1 twin), int8 as the W8A8 tier
    if ((profile & (BACKEND_PROFILE_EXACT | BACKEND_PROFILE_FMA)) && G.kind == kKindRwkv &&
        ((profile & (BACKEND_PROFILE_FMA | BACKEND_PROFILE_W8A8)) || (profile & 3) != 0)) {
        log("RWKV-7's reference-order tier is F32 in numeric contract 1 (profile 64); its int8 one is the W8A8 tier");
        free_model();
        return BACKEND_INIT_FAILED;
    }
    if ((profile & BACKEND_PROFILE_W8A8) && (G.kind != kKindRwkv || (profile & 3) != BACKEND_PROFILE_Q8_ROW)) {
        log("the W8A8 tier serves RWKV-7 with per-row int8 weights only");
        free_model();
        return BACKEND_INIT_FAILED;
    }
    const int lr = G.kind == kKindRwkv ? load_rwkv(path, profile) : load_weights(path, profile);
    if (lr != 0) {
        free_model();
        return lr == -2 ? BACKEND_INIT_FAILED : BACKEND_WEIGHTS_NOT_FOUND;
    }
    if (hipMalloc((void**)&G.d_err, sizeof(uint32_t)) != hipSuccess) {
        G.d_err = nullptr;
        free_model();
        return BACKEND_INIT_FAILED;
    }
    G.allocs.push_back(G.d_err);
    if (hipMemset(G.d_err, 0, sizeof(uint32_t)) != hipSuccess || !pool_alloc(G.v1, 1)) {
        free_model();
        return BACKEND_INIT_FAILED;
    }
    G.ready = true;
    memset(info_out, 0, sizeof(*info_out));
    info_out->ffi_version = BACKEND_FFI_VERSION;
    info_out->vocab_size = G.dims.vocab;
    info_out->hidden_dim = G.dims.d;
    static const char* names[2][3] = {{"hip-gfx950-mamba-f32", "hip-gfx950-mamba-q8", "hip-gfx950-mamba-q8row"},
                                       {"hip-gfx950-rwkv7-f32", "hip-gfx950-rwkv7-q8", "hip-gfx950-rwkv7-q8row"}};
    static const char* exact_names[2][3] = {
        {"hip-gfx950-mamba-f32-ref", "hip-gfx950-mamba-q8-ref", "hip-gfx950-mamba-q8row-ref"},
        {"hip-gfx950-mamba-f32-ref-fma", "hip-gfx950-mamba-q8-ref-fma", "hip-gfx950-mamba-q8row-ref-fma"}};
    const char* name = G.r_a8      ? "hip-gfx950-rwkv7-w8a8"
                       : G.r_exact ? "hip-gfx950-rwkv7-f32-ref"
                       : G.exact   ? exact_names[G.exact_fma ? 1 : 0][profile & 3]
                                 : names[G.kind == kKindRwkv ? 1 : 0][profile & 3];
    memcpy(info_out->name, name, strlen(name));
    size_t fr = 0, tot = 0;
    (void)hipMemGetInfo(&fr, &tot);
    log("ready: vocab=%u d_model=%u n_layer=%u abi=%d | GPU %.0f/%.0f MB used", G.dims.vocab, G.dims.d, G.dims.nl,
        BACKEND_ABI_VERSION, (tot - fr) / 1048576.0, tot / 1048576.0);
    return BACKEND_OK;
}

}  // namespace
}  // namespace rdk

using namespace rdk;

namespace {
// The portable element-wise functions on the device (redukt_backend_eval_math).
__global__ void k_eval_math(uint32_t fn, const float* __restrict__ x, float* __restrict__ y, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    float r;
    switch (fn) {
        case 0: r = exp_f(v); break;
        case 1: r = lane_exp_f(v); break;
        case 2: r = ln_f(v); break;
        case 3: r = softplus_f(v); break;
        case 4: r = lane_sigmoid_f(v); break;
        default: r = 1.0f / (1.0f + exp_f(-v)); break;
    }
    y[i] = r;
}

// The copy of redukt_backend_copy_probe: W bytes per lane per load and store, cache policy
// AUX (0 default, 2 streaming), a grid-stride loop over buffer descriptors of the exact size.
template <int AUX, int W>
__global__ __launch_bounds__(256) void k_copy_probe(const void* src, void* dst, uint32_t bytes) {
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(src), (short)0, (int)bytes, 0x00020000);
    const auto rd = __builtin_amdgcn_make_buffer_rsrc(dst, (short)0, (int)bytes, 0x00020000);
    const uint32_t stride = gridDim.x * blockDim.x * W;
    for (uint32_t o = (blockIdx.x * blockDim.x + threadIdx.x) * W; o < bytes; o += stride) {
        if constexpr (W == 16)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_amdgcn_raw_buffer_load_b128(rs, (int)o, 0, AUX), rd, (int)o,
                                                   0, AUX);
        else
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_amdgcn_raw_buffer_load_b32(rs, (int)o, 0, AUX), rd, (int)o,
                                                  0, AUX);
    }
}
}  // namespace

extern "C" {

BackendResult redukt_backend_init(const uint8_t* weights_path, int32_t device_id, BackendInfo* info_out) {
    return (BackendResult)init_common(weights_path, device_id, env_profile(), info_out);
}

BackendResult redukt_backend_forward(uint32_t token, float* out_logits, uint32_t vocab_size) {
    if (!G.ready || !out_logits || vocab_size != G.dims.vocab) return BACKEND_FORWARD_FAILED;
    const uint32_t slot = 0;
    return pool_forward(G.v1, 1, &slot, &token, out_logits, false) == BACKEND_OK ? BACKEND_OK
                                                                                   : BACKEND_FORWARD_FAILED;
}

void redukt_backend_reset_state(void) {
    if (!G.ready) return;
    const uint32_t slot = 0;
    if (pool_reset(G.v1, 1, &slot) != BACKEND_OK) log("reset_state failed");
}

void redukt_backend_free(void) {
    free_model();
    log("freed");
}

uint32_t redukt_backend_abi_version(void) { return BACKEND_ABI_VERSION; }

int32_t redukt_backend_batch_init(uint32_t max_streams) {
    if (!G.ready) return BACKEND_INIT_FAILED;
    if (max_streams > BACKEND_MAX_STREAMS) return BACKEND_INVALID_ARGUMENT;
    if (hipStreamSynchronize(G.stream) != hipSuccess) return BACKEND_INIT_FAILED;
    G.runner.clear();
    pool_free(G.batch);
    if (max_streams == 0) return BACKEND_OK;
    if (!pool_alloc(G.batch, max_streams)) {
        pool_free(G.batch);
        return BACKEND_INIT_FAILED;
    }
    log("batch pool: %u streams", max_streams);
    return BACKEND_OK;
}

int32_t redukt_backend_batch_reset(const uint32_t* slots, uint32_t n_slots) {
    if (!G.ready || G.batch.cap == 0) return BACKEND_INIT_FAILED;
    if (!slots) return pool_reset(G.batch, G.batch.cap, nullptr);
    if (n_slots > G.batch.cap) return BACKEND_INVALID_ARGUMENT;
    return pool_reset(G.batch, n_slots, slots);
}

static int32_t forward_batch_impl(uint32_t n, const uint32_t* slots, const uint32_t* tokens, float* out,
                                  uint32_t vocab_size, bool probs) {
    if (!G.ready || G.batch.cap == 0) return BACKEND_INIT_FAILED;
    if (vocab_size != G.dims.vocab || n > G.batch.cap) return BACKEND_INVALID_ARGUMENT;
    if (n == 0) return BACKEND_OK;
    if (!slots || !tokens || !out) return BACKEND_INVALID_ARGUMENT;
    return pool_forward(G.batch, n, slots, tokens, out, probs);
}

int32_t redukt_backend_forward_batch(uint32_t n_streams, const uint32_t* slots, const uint32_t* tokens,
                                     float* out_logits, uint32_t vocab_size) {
    return forward_batch_impl(n_streams, slots, tokens, out_logits, vocab_size, false);
}

int32_t redukt_backend_init_ex(const uint8_t* weights_path, int32_t device_id, uint32_t profile,
                               BackendInfo* info_out) {
    if (profile > 255u) return BACKEND_INVALID_ARGUMENT;   // bits 0-7
    return init_common(weights_path, device_id, profile, info_out);
}

int32_t redukt_backend_forward_batch_probs(uint32_t n_streams, const uint32_t* slots, const uint32_t* tokens,
                                           float* out_probs, uint32_t vocab_size) {
    return forward_batch_impl(n_streams, slots, tokens, out_probs, vocab_size, true);
}

// ---------------------------------------------------------------- CDFs on the device
// The CDF kernels' scratch (exp values and the two sums per row) and, for the host-buffer
// entry point, the CDF rows themselves: one allocation, grown on demand (the stream is
// synchronized before the old one is freed).
bool cdf_space(uint32_t rows, uint32_t n, bool with_out, void** scratch, uint32_t** out, uint32_t** pick = nullptr) {
    const size_t sb = (cdf_scratch_bytes(rows, n) + 255) & ~(size_t)255;
    const size_t ob = with_out ? ((size_t)rows * (n + 1) * 4 + 255) & ~(size_t)255 : 0;
    // pick: the coder's three or four values per row
    const size_t need = sb + ob + (pick ? (size_t)rows * 4 * 4 : 0);
    if (need > G.cdf_bytes) {
        if (G.cdf_mem) {
            if (hipStreamSynchronize(G.stream) != hipSuccess) return false;
            (void)hipFree(G.cdf_mem);
            G.cdf_mem = nullptr;
            G.cdf_bytes = 0;
        }
        if (hipMalloc(&G.cdf_mem, need) != hipSuccess) {
            G.cdf_mem = nullptr;
            return false;
        }
        G.cdf_bytes = need;
    }
    *scratch = G.cdf_mem;
    if (out) *out = (uint32_t*)((unsigned char*)G.cdf_mem + sb);
    if (pick) *pick = (uint32_t*)((unsigned char*)G.cdf_mem + sb + ob);
    return true;
}

int32_t redukt_backend_forward_batch_cdf(uint32_t n_streams, const uint32_t* slots, const uint32_t* tokens,
                                         uint32_t* out_cdf, uint32_t cdf_len) {
    if (!G.ready || G.batch.cap == 0) return BACKEND_INIT_FAILED;
    const uint32_t V = G.kind == kKindRwkv ? G.rdims.vocab : G.dims.vocab;
    if (cdf_len != V + 1 || n_streams > G.batch.cap || V >= (1u << 24)) return BACKEND_INVALID_ARGUMENT;
    if (n_streams == 0) return BACKEND_OK;
    if (!slots || !tokens || !out_cdf) return BACKEND_INVALID_ARGUMENT;
    Pool& p = G.batch;
    memset(p.seen, 0, p.cap);
    for (uint32_t b = 0; b < n_streams; b++) {
        if (slots[b] >= p.cap || p.seen[slots[b]] || tokens[b] >= V) return BACKEND_INVALID_ARGUMENT;
        p.seen[slots[b]] = 1;
    }
    void* scratch = nullptr;
    uint32_t* d_cdf = nullptr;
    if (!cdf_space(n_streams, V, true, &scratch, &d_cdf)) return BACKEND_FORWARD_FAILED;
    memcpy(p.h_slots, slots, sizeof(uint32_t) * n_streams);
    memcpy(p.h_slots + n_streams, tokens, sizeof(uint32_t) * n_streams);
    if (hipMemcpyAsync(p.d_slots, p.h_slots, sizeof(uint32_t) * 2 * n_streams, hipMemcpyHostToDevice, G.stream) !=
        hipSuccess)
        return BACKEND_FORWARD_FAILED;
    if (run_step(p, n_streams, p.d_slots, p.d_slots + n_streams, p.out, false, false) != hipSuccess ||
        cdf_launch(p.out, n_streams, V, scratch, d_cdf, G.stream) != hipSuccess)
        return BACKEND_FORWARD_FAILED;
    if (!copy_out(p, out_cdf, d_cdf, sizeof(uint32_t) * n_streams * (size_t)(V + 1))) return BACKEND_FORWARD_FAILED;
    return BACKEND_OK;
}

namespace {
// forward_batch_cdf_sym and _find: one H2D copy of the slots, the tokens and each stream's
// next symbol (sym) or decoder target (find) through the pool's pinned staging; the step,
// the device CDF and the kernel that reads the rows; `per` u32 a stream back through the
// pinned output staging, waited for by polling its event.
int32_t forward_batch_cdf_read(uint32_t n_streams, const uint32_t* slots, const uint32_t* tokens,
                               const uint32_t* third, uint32_t* out, uint32_t vocab_size, bool find) {
    if (!G.ready || G.batch.cap == 0) return BACKEND_INIT_FAILED;
    const uint32_t V = G.kind == kKindRwkv ? G.rdims.vocab : G.dims.vocab;
    if (vocab_size != V || n_streams > G.batch.cap || V >= (1u << 24)) return BACKEND_INVALID_ARGUMENT;
    if (n_streams == 0) return BACKEND_OK;
    if (!slots || !tokens || !third || !out) return BACKEND_INVALID_ARGUMENT;
    Pool& p = G.batch;
    memset(p.seen, 0, p.cap);
    for (uint32_t b = 0; b < n_streams; b++) {
        if (slots[b] >= p.cap || p.seen[slots[b]] || tokens[b] >= V || (!find && third[b] >= V))
            return BACKEND_INVALID_ARGUMENT;
        p.seen[slots[b]] = 1;
    }
    const size_t per = find ? 4 : 3;
    const size_t out_bytes = sizeof(uint32_t) * per * n_streams;
    if (out_bytes > p.out_stage_bytes) return BACKEND_FORWARD_FAILED;   // staging holds >= 4 u32 a stream
    void* scratch = nullptr;
    uint32_t *d_cdf = nullptr, *d_out = nullptr;
    if (!cdf_space(n_streams, V, true, &scratch, &d_cdf, &d_out)) return BACKEND_FORWARD_FAILED;
    memcpy(p.h_slots, slots, sizeof(uint32_t) * n_streams);
    memcpy(p.h_slots + n_streams, tokens, sizeof(uint32_t) * n_streams);
    memcpy(p.h_slots + 2 * n_streams, third, sizeof(uint32_t) * n_streams);
    if (hipMemcpyAsync(p.d_slots, p.h_slots, sizeof(uint32_t) * 3 * n_streams, hipMemcpyHostToDevice, G.stream) !=
        hipSuccess)
        return BACKEND_FORWARD_FAILED;
    const uint32_t* d_third = p.d_slots + 2 * n_streams;
    if (run_step(p, n_streams, p.d_slots, p.d_slots + n_streams, p.out, false, false) != hipSuccess ||
        cdf_launch(p.out, n_streams, V, scratch, d_cdf, G.stream) != hipSuccess ||
        (find ? cdf_find_launch(d_cdf, n_streams, V, d_third, d_out, G.stream)
              : cdf_pick_launch(d_cdf, n_streams, V, d_third, d_out, G.stream)) != hipSuccess)
        return BACKEND_FORWARD_FAILED;
    if (hipMemcpyAsync(p.h_out, d_out, out_bytes, hipMemcpyDeviceToHost, G.stream) != hipSuccess ||
        hipEventRecord(p.out_ev[0], G.stream) != hipSuccess || !event_wait(p.out_ev[0]))
        return BACKEND_FORWARD_FAILED;
    memcpy(out, p.h_out, out_bytes);
    return BACKEND_OK;
}
}  // namespace

int32_t redukt_backend_forward_batch_cdf_sym(uint32_t n_streams, const uint32_t* slots, const uint32_t* tokens,
                                             const uint32_t* next_syms, uint32_t* out_bounds, uint32_t vocab_size) {
    return forward_batch_cdf_read(n_streams, slots, tokens, next_syms, out_bounds, vocab_size, false);
}

// Tickets of queued calls, never reused in the process (a ticket from before a batch_init
// is refused, not matched to a later call).
static uint64_t g_next_ticket = 1;

int32_t redukt_backend_forward_batch_cdf_sym_submit(uint32_t n_streams, const uint32_t* slots, const uint32_t* tokens,
                                                    const uint32_t* next_syms, uint32_t vocab_size, uint64_t* ticket) {
    if (!G.ready || G.batch.cap == 0) return BACKEND_INIT_FAILED;
    const uint32_t V = G.kind == kKindRwkv ? G.rdims.vocab : G.dims.vocab;
    if (!ticket || vocab_size != V || n_streams > G.batch.cap || V >= (1u << 24)) return BACKEND_INVALID_ARGUMENT;
    if (n_streams > 0 && (!slots || !tokens || !next_syms)) return BACKEND_INVALID_ARGUMENT;
    Pool& p = G.batch;
    Pool::Queued* q = nullptr;
    for (Pool::Queued& c : p.queued)
        if (c.ticket == 0) {
            q = &c;
            break;
        }
    if (!q) return BACKEND_INVALID_ARGUMENT;   // Pool::kQueued calls in flight: wait for one first
    memset(p.seen, 0, p.cap);
    for (uint32_t b = 0; b < n_streams; b++) {
        if (slots[b] >= p.cap || p.seen[slots[b]] || tokens[b] >= V || next_syms[b] >= V) return BACKEND_INVALID_ARGUMENT;
        p.seen[slots[b]] = 1;
    }
    if (n_streams > 0) {
        void* scratch = nullptr;
        uint32_t *d_cdf = nullptr, *d_pick = nullptr;
        // (a regrown scratch synchronizes the stream first, the other call's work included)
        if (!cdf_space(n_streams, V, true, &scratch, &d_cdf, &d_pick)) return BACKEND_FORWARD_FAILED;
        memcpy(q->h_in, slots, sizeof(uint32_t) * n_streams);
        memcpy(q->h_in + n_streams, tokens, sizeof(uint32_t) * n_streams);
        memcpy(q->h_in + 2 * n_streams, next_syms, sizeof(uint32_t) * n_streams);
        const bool ok =
            hipMemcpyAsync(q->d_in, q->h_in, sizeof(uint32_t) * 3 * n_streams, hipMemcpyHostToDevice, G.stream) ==
                hipSuccess &&
            run_step(p, n_streams, q->d_in, q->d_in + n_streams, p.out, false, false) == hipSuccess &&
            cdf_launch(p.out, n_streams, V, scratch, d_cdf, G.stream) == hipSuccess &&
            cdf_pick_launch(d_cdf, n_streams, V, q->d_in + 2 * n_streams, d_pick, G.stream) == hipSuccess &&
            hipMemcpyAsync(q->h_res, d_pick, sizeof(uint32_t) * 3 * n_streams, hipMemcpyDeviceToHost, G.stream) ==
                hipSuccess;
        if (!ok) {
            // what was queued finishes before its buffers can be reused
            (void)hipStreamSynchronize(G.stream);
            return BACKEND_FORWARD_FAILED;
        }
    }
    if (hipEventRecord(q->done, G.stream) != hipSuccess) {
        (void)hipStreamSynchronize(G.stream);
        return BACKEND_FORWARD_FAILED;
    }
    q->n = n_streams;
    q->ticket = g_next_ticket++;
    *ticket = q->ticket;
    return BACKEND_OK;
}

int32_t redukt_backend_forward_batch_cdf_sym_wait(uint64_t ticket, uint32_t* out_bounds, uint32_t n_streams) {
    if (!G.ready || G.batch.cap == 0) return BACKEND_INIT_FAILED;
    Pool::Queued* q = nullptr;
    for (Pool::Queued& c : G.batch.queued)
        if (ticket != 0 && c.ticket == ticket) q = &c;
    if (!q || n_streams != q->n || (n_streams > 0 && !out_bounds)) return BACKEND_INVALID_ARGUMENT;
    const bool ok = event_wait(q->done);
    if (ok) memcpy(out_bounds, q->h_res, sizeof(uint32_t) * 3 * n_streams);
    q->ticket = 0;
    q->n = 0;
    return ok ? BACKEND_OK : BACKEND_FORWARD_FAILED;
}

int32_t redukt_backend_forward_batch_cdf_find(uint32_t n_streams, const uint32_t* slots, const uint32_t* tokens,
                                              const uint32_t* targets, uint32_t* out_found, uint32_t vocab_size) {
    return forward_batch_cdf_read(n_streams, slots, tokens, targets, out_found, vocab_size, true);
}

int32_t redukt_backend_cdf_from_logits_device(const float* d_logits, uint32_t rows, uint32_t n, uint32_t* d_cdf) {
    if (!G.ready) return BACKEND_INIT_FAILED;
    if (n == 0 || n >= (1u << 24) || (rows > 0 && (!d_logits || !d_cdf))) return BACKEND_INVALID_ARGUMENT;
    if (rows == 0) return BACKEND_OK;
    void* scratch = nullptr;
    if (!cdf_space(rows, n, false, &scratch, nullptr)) return BACKEND_FORWARD_FAILED;
    return cdf_launch(d_logits, rows, n, scratch, d_cdf, G.stream) == hipSuccess ? BACKEND_OK : BACKEND_FORWARD_FAILED;
}

int32_t redukt_backend_forward_batch_device(uint32_t n_streams, const uint32_t* d_slots, const uint32_t* d_tokens,
                                            float* d_out, uint32_t vocab_size, uint32_t flags) {
    if (!G.ready || G.batch.cap == 0) return BACKEND_INIT_FAILED;
    if (vocab_size != G.dims.vocab || n_streams > G.batch.cap) return BACKEND_INVALID_ARGUMENT;
    if (n_streams == 0) return BACKEND_OK;
    if (!d_slots || !d_tokens || !d_out) return BACKEND_INVALID_ARGUMENT;
    return run_step(G.batch, n_streams, d_slots, d_tokens, d_out, (flags & 1u) != 0, true) == hipSuccess
               ? BACKEND_OK
               : BACKEND_FORWARD_FAILED;
}

int32_t redukt_backend_forward_batch_device_noalloc(uint32_t n_streams, const uint32_t* d_slots,
                                                    const uint32_t* d_tokens, float* d_out, uint32_t vocab_size,
                                                    uint32_t flags) {
    if (!G.ready || G.batch.cap == 0) return BACKEND_INIT_FAILED;
    if (G.kind != kKindMamba || vocab_size != G.dims.vocab || n_streams > G.batch.cap) return BACKEND_INVALID_ARGUMENT;
    if (n_streams == 0) return BACKEND_OK;
    if (!d_slots || !d_tokens || !d_out) return BACKEND_INVALID_ARGUMENT;
    unsigned char* base = G.device < kMaxDevices ? (unsigned char*)g_noalloc_base[G.device] : nullptr;
    if (!base) return BACKEND_INIT_FAILED;
    Pool v;
    size_t used = 0;
    if (!noalloc_view(v, n_streams, base, &used)) {
        log("forward_batch_device_noalloc: %u streams need %zu bytes of scratch, more than %zu", n_streams, used,
            kNoAllocScratchBytes);
        return BACKEND_INVALID_ARGUMENT;
    }
    const size_t n16 = used / 16;
    hipLaunchKernelGGL(k_clear, dim3((unsigned)std::min<size_t>((n16 + 255) / 256, 1024)), dim3(256), 0, G.stream,
                       (uint4*)base, n16);
    if (hipGetLastError() != hipSuccess) return BACKEND_FORWARD_FAILED;
    StepIO io{n_streams, d_slots, d_tokens, d_out, (flags & 1u) != 0, true, G.d_err};
    if (G.gemv) {
        const GemvStep src(gemv_view());
        return G.runner.run_direct(src, v, io, G.stream) == hipSuccess ? BACKEND_OK : BACKEND_FORWARD_FAILED;
    }
    if (G.exact) {
        const ExactStep src(exact_view());
        return G.runner.run_direct(src, v, io, G.stream) == hipSuccess ? BACKEND_OK : BACKEND_FORWARD_FAILED;
    }
    const MambaStep src(model_view());
    return G.runner.run_direct(src, v, io, G.stream) == hipSuccess ? BACKEND_OK : BACKEND_FORWARD_FAILED;
}

int32_t redukt_backend_device_status(void) {
    if (!G.ready) return BACKEND_INIT_FAILED;
    uint32_t err = 0;
    if (hipMemcpyAsync(&err, G.d_err, sizeof(err), hipMemcpyDeviceToHost, G.stream) != hipSuccess ||
        hipStreamSynchronize(G.stream) != hipSuccess)
        return BACKEND_FORWARD_FAILED;
    if (err) {
        const uint32_t zero = 0;
        if (hipMemcpy(G.d_err, &zero, sizeof(zero), hipMemcpyHostToDevice) != hipSuccess) return BACKEND_FORWARD_FAILED;
        // bits 0-1: a bad slot or token, a repeated slot; above: the persistent step
        // kernel gave up waiting for a phase or ran on an unexpected XCD
        return (err & ~3u) ? BACKEND_FORWARD_FAILED : BACKEND_INVALID_ARGUMENT;
    }
    return BACKEND_OK;
}

void* redukt_backend_stream(void) { return (void*)G.stream; }

int32_t redukt_backend_probe_kernel(uint32_t kernel_class, void** events, uint32_t n_events) {
    if (!G.ready) return BACKEND_INIT_FAILED;
    const bool only = (kernel_class & REDUKT_PROBE_CLASS_ONLY) != 0;
    kernel_class &= ~REDUKT_PROBE_CLASS_ONLY;
    if (kernel_class >= KC_COUNT || (kernel_class != KC_NONE && (!events || n_events < 2)))
        return BACKEND_INVALID_ARGUMENT;
    G.probe = Probe{};
    if (kernel_class != KC_NONE) {
        G.probe.cls = kernel_class;
        G.probe.only = only;
        G.probe.ev = (hipEvent_t*)events;
        G.probe.cap = n_events;
    }
    return BACKEND_OK;
}

uint32_t redukt_backend_probe_used(void) { return G.probe.used; }

int32_t redukt_backend_get_rwkv_state(uint32_t slot, uint32_t layer, float* x_att, float* wkv, float* x_ffn) {
    if (!G.ready || G.batch.cap == 0) return BACKEND_INIT_FAILED;
    if (G.kind != kKindRwkv || slot >= G.batch.cap || layer >= G.rdims.nl) return BACKEND_INVALID_ARGUMENT;
    if (hipStreamSynchronize(G.stream) != hipSuccess) return BACKEND_FORWARD_FAILED;
    const RDims& R = G.rdims;
    const size_t d = R.d, wl = (size_t)R.h * R.n * R.n, row = (size_t)slot * R.nl + layer;
    const Pool& p = G.batch;
    if (x_att && hipMemcpy(x_att, p.x_att + row * d, d * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return BACKEND_FORWARD_FAILED;
    if (wkv) {
        // the pool holds each head as [j / 4][i][4]; the caller gets [head][i][j]
        std::vector<float> t(wl);
        if (hipMemcpy(t.data(), p.wkv + row * wl, wl * 4, hipMemcpyDeviceToHost) != hipSuccess) return BACKEND_FORWARD_FAILED;
        const size_t n = R.n;
        for (size_t hh = 0; hh < R.h; hh++)
            for (size_t i = 0; i < n; i++)
                for (size_t j = 0; j < n; j++)
                    wkv[(hh * n + i) * n + j] = t[hh * n * n + ((j / 4) * n + i) * 4 + j % 4];
    }
    if (x_ffn && hipMemcpy(x_ffn, p.x_ffn + row * d, d * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return BACKEND_FORWARD_FAILED;
    return BACKEND_OK;
}

int32_t redukt_backend_get_state(uint32_t slot, uint32_t layer, float* conv_out, float* ssm_out) {
    if (!G.ready || G.batch.cap == 0) return BACKEND_INIT_FAILED;
    if (G.kind != kKindMamba) return BACKEND_INVALID_ARGUMENT;
    if (slot >= G.batch.cap || layer >= G.dims.nl) return BACKEND_INVALID_ARGUMENT;
    if (hipStreamSynchronize(G.stream) != hipSuccess) return BACKEND_FORWARD_FAILED;
    const size_t cl = (size_t)G.dims.di * (G.dims.dc - 1), sl = (size_t)G.dims.di * 16;
    const Pool& p = G.batch;
    if (conv_out && hipMemcpy(conv_out, p.conv + ((size_t)layer * p.scap + slot) * cl, cl * 4, hipMemcpyDeviceToHost) !=
                        hipSuccess)
        return BACKEND_FORWARD_FAILED;
    if (ssm_out) {
        // the pool holds [16][di] per slot; the caller gets [di][16]
        std::vector<float> sm(sl);
        if (hipMemcpy(sm.data(), p.ssm + ((size_t)layer * p.scap + slot) * sl, sl * 4, hipMemcpyDeviceToHost) !=
            hipSuccess)
            return BACKEND_FORWARD_FAILED;
        const size_t di = G.dims.di;
        for (size_t j = 0; j < di; j++)
            for (size_t n = 0; n < 16; n++) ssm_out[j * 16 + n] = sm[n * di + j];
    }
    return BACKEND_OK;
}

int32_t redukt_backend_eval_math(uint32_t fn, const float* x, float* y, uint32_t n) {
    if (fn >= REDUKT_MATH_FN_COUNT || (n && (!x || !y))) return BACKEND_INVALID_ARGUMENT;
    if (n == 0) return BACKEND_OK;
    float* d = nullptr;
    const size_t bytes = sizeof(float) * n;
    if (hipMalloc(&d, 2 * bytes) != hipSuccess) return BACKEND_FORWARD_FAILED;
    hipError_t e = hipMemcpy(d, x, bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(k_eval_math, dim3((n + 255) / 256), dim3(256), 0, 0, fn, d, d + n, n);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(y, d + n, bytes, hipMemcpyDeviceToHost);
    (void)hipFree(d);
    return e == hipSuccess ? BACKEND_OK : BACKEND_FORWARD_FAILED;
}

int32_t redukt_backend_copy_probe(void* dst, const void* src, uint64_t bytes, uint32_t mode) {
    if (mode > 3 || bytes % 16 || bytes >= (1ull << 31) || (bytes && (!dst || !src))) return BACKEND_INVALID_ARGUMENT;
    if (bytes == 0) return BACKEND_OK;
    const hipStream_t st = G.ready ? G.stream : nullptr;
    const uint32_t b = (uint32_t)bytes;
    const void* fns[4] = {(const void*)k_copy_probe<0, 4>, (const void*)k_copy_probe<2, 4>,
                          (const void*)k_copy_probe<0, 16>, (const void*)k_copy_probe<2, 16>};
    void* args[] = {(void*)&src, (void*)&dst, (void*)&b};
    return hipLaunchKernel(fns[mode], dim3(1024), dim3(256), args, 0, st) == hipSuccess ? BACKEND_OK
                                                                                      : BACKEND_FORWARD_FAILED;
}

}  // extern "C"
