// model.h — device-side model and state-pool layout shared by the host code and the
// kernels of libredukt_gpu.so.
#pragma once
// No a*b+c in this file may be fused: the element-wise arithmetic follows the
// reference operation by operation (a header is compiled before its includer's pragmas).
#pragma clang fp contract(off)

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

#include "step.h"

namespace rdk {

constexpr int kRowTile = 16;   // MFMA M and N
constexpr int kKStep = 32;     // MFMA K of v_mfma_f32_16x16x32_bf16
constexpr int kKAlign = 64;    // column padding: k-steps come in pairs

// A projection matrix resident in HBM, pre-tiled for v_mfma_f32_16x16x32_bf16.
// Rows are padded to whole 16-row tiles and columns to whole pairs of 32-column k-steps
// (zeros).  For row tile t and k-step s, lane l of a wavefront owns the A fragment
// W[16t + l%16][32s + 8(l/16) .. +8]:
//   F32: [t][s][lane][8 f32]                 — 32 bytes per lane and k-step
//   Q8 : [t][s/2][lane][s%2][8 int8]         — 16 bytes per lane and k-step pair
// so every fragment load of a wavefront is one contiguous run (2 KB / 1 KB).
// Q8 scales: group == cols: one per row, [rt*16]; otherwise (64 columns per scale)
// [rt*16][ks/2].
struct TMat {
    int rows = 0, cols = 0;
    int rt = 0, ks = 0;   // row tiles, k-steps (even)
    int group = 0;        // 0: F32; Q8: columns per scale
    void* w = nullptr;
    float* scales = nullptr;
    size_t bytes() const;  // HBM bytes of weights + scales as stored
};

// A projection matrix in the layout of the wavefront-GEMV kernels (the small-batch tier).
// K = cols is cut into 16-element chunks, CR = K / 16 per row.  A wave multiplies RPI rows
// at a time (an iteration block); lane l owns row l % RPI of the block and the CPL chunks
// c_j = l / RPI + (64 / RPI) j, j < CPL, so CPL * 64 = CR * RPI.  The lane's activation
// slice (its chunks' K indices) is therefore the same for every block, and every load of
// a wave is one contiguous run: block i, load j, lane l at ((i CPL + j) 64 + l) * chunk
// bytes (Q8: 16 int8, F32: 16 f32).  Rows are padded to whole blocks with zeros.  Q8
// scales are one per row ([rows]).
struct GMat {
    int rows = 0, cols = 0;
    int rpi = 0, cpl = 0, blocks = 0;
    bool q8 = false;
    void* w = nullptr;
    float* scales = nullptr;
    size_t bytes() const;
};

// A row-major [rows][cols] matrix for the reference-order tier: F32, or int8 with one f32
// scale per `group` columns ([rows][cols / group]), the layout of the reference's own
// Q8wMatrix (src/domain/gemv.rs:244-273).
struct RowMat {
    int rows = 0, cols = 0;
    int group = 0;        // 0: F32; Q8: columns per scale
    void* w = nullptr;
    float* scales = nullptr;
    size_t bytes() const { return w ? (size_t)rows * cols * (group ? 1 : 4) + (group ? (size_t)rows * (cols / group) * 4 : 0) : 0; }
};

struct DLayer {
    float* norm_w = nullptr;
    float* norm_b = nullptr;   // LayerNorm bias (flags bit 0) or null
    TMat in_x, in_z;           // in_proj rows [0, di) (conv branch) and [di, 2di) (gate)
    TMat x_proj;               // [dr + 2*ds][di]
    TMat out_proj;             // [d][di]
    float* conv_w = nullptr;   // [di][dc]
    float* conv_b = nullptr;   // [di]
    // dt_proj row-major with rows padded to dt_pad (a multiple of 16) columns, so thread j
    // loads its row with 16-byte vector loads.  F32 in dt_w, or Q8 in dt_q with one scale
    // per row in dt_scales.
    float* dt_w = nullptr;
    int8_t* dt_q = nullptr;
    float* dt_scales = nullptr;
    int dt_pad = 0;
    float* dt_b = nullptr;     // [di]
    float* a_exp = nullptr;    // [16][di] (state-major): exp(A_log), constant per load
    float* d_vec = nullptr;    // [di]
    // The wavefront-GEMV tier (weight profile bit 4): in_proj rows [0, 2 di) and out_proj in
    // GEMV layout, x_proj row-major [xr][di] (F32 in xp_w, or Q8 in xp_q with one scale per
    // row in xp_scales); dt_proj as above.
    GMat g_in, g_out;
    RowMat e_in, e_xp, e_out;  // the reference-order tier's in_proj, x_proj and out_proj
    float* xp_w = nullptr;
    int8_t* xp_q = nullptr;
    float* xp_scales = nullptr;
};

struct Dims {
    uint32_t vocab = 0, d = 0, di = 0, ds = 0, dc = 0, dr = 0, nl = 0, flags = 0, tokenizer = 0;
    uint32_t xr() const { return dr + 2 * ds; }
};

// Recurrent state of `cap` slots plus the per-step scratch of `cap` batch rows.
// The step's validated slot list (Pool::slots) is allocated in whole blocks of this many
// words: a kernel may read the slot words of its whole stream chunk with scalar loads, past
// the last stream of a ragged chunk too (those words only feed streams never stored).
constexpr uint32_t kSlotWordAlign = 64;

// State: conv [layer][slot][di][dc-1] and ssm [layer][slot][16][di] f32 over scap slots (state-major, so
// the scan's loads of one state index over 64 channels are contiguous); one slot's state
// of one layer is one contiguous run either way (18 KB + 96 KB at Mamba-130M).
struct Pool {
    uint32_t cap = 0;
    // State slots: cap + 1.  Slot `cap` is a scratch slot no caller can name: a
    // device-checked step (forward_batch_device) routes every invalid entry and every
    // repeat of a slot already listed earlier in the batch there, so a bad entry never
    // touches a real slot and no two streams of a step share one.
    uint32_t scap = 0;
    uint32_t gcap = 0;           // stream groups of 16 covering cap
    uint32_t xcap = 0;           // batch rows of the x_proj partials (their row stride; cap unless carved smaller)
    void* block = nullptr;       // the one device allocation all device arrays below are carved from
    float* conv = nullptr;
    float* ssm = nullptr;
    float* x = nullptr;          // [cap][d] residual stream
    float* u = nullptr;          // [cap][di] conv + SiLU output
    float* z = nullptr;          // [cap][di] gate branch
    float* xpart = nullptr;      // [di/64][cap][xr_pad] split-K partials of x_proj
    __bf16* glimb = nullptr;     // [gcap][di/32][3][64][8] gated, 3 bf16 limbs, B-fragment tiles
    float* g32 = nullptr;        // [cap][di] gated, f32 (the wavefront-GEMV and reference-order tiers)
    float* normed = nullptr;     // [cap][d] a norm's output (the reference-order tier)
    // Next projection's input, written by the producer of the residual stream (embedding,
    // out_proj): x * norm_w as 3 bf16 limbs in B-fragment tiles, [gcap][ks_d][3][64][8]
    // with ks_d = the k-steps of a d-column projection, plus per-16-column partial sums of
    // x^2, [cap][d/16], from which the consumer forms the RMS scale of each stream.
    __bf16* xw = nullptr;
    float* ssp = nullptr;
    // RWKV-7 (allocated for RWKV-7 models only)
    float* x_att = nullptr;      // [slot][layer][d] time-mix token-shift input (ln1 output)
    float* x_ffn = nullptr;      // [slot][layer][d] channel-mix token-shift input (ln2 output)
    float* wkv = nullptr;        // [slot][layer][head][j / 4][i][4] WKV-7 state S[i][j] (row i, column j)
    float* vfirst = nullptr;     // [cap][d] layer-0 value of the current token, per batch position
    float* rkv = nullptr;        // [cap][3d] receptance, key, value
    float* lorad = nullptr;      // [cap][4d] second LoRA stages: decay, a, g, v
    __bf16* mixl = nullptr;      // 6 x [gcap][ks_d][3][64][8]: x_r, x_w, x_k, x_v, x_a, x_g inputs
    __bf16* loral = nullptr;     // 4 x [gcap][ks_lora][3][64][8]: tanh(w1·x), a1·x, sigmoid(g1·x), v1·x
    __bf16* gatedl = nullptr;    // [gcap][ks_d][3][64][8] gated WKV output
    __bf16* ffnl = nullptr;      // [gcap][ks_d][3][64][8] channel-mix input
    __bf16* actl = nullptr;      // [gcap][ks_ffn][3][64][8] squared-ReLU activations
    __bf16* headl = nullptr;     // [gcap][ks_d][3][64][8] final LayerNorm output
    // RWKV-7 W8A8 tier (instead of the limb buffers above)
    float* mixf = nullptr;       // [4][cap][d] LoRA inputs x_w, x_a, x_g, x_v (f32); reference-order tier: [6][cap][d], then x_r, x_k
    float* lorah = nullptr;      // [cap][sum of ranks] first LoRA stages after their activation
    int8_t* aq = nullptr;        // int8 activations, kAqAct x [rows16][dp], then [rows16][fp]
    float* as = nullptr;         // their scales, kAqVecs x [cap]
    float* gatedf = nullptr;     // [rows16][dp] gated WKV output (f32)
    float* actf = nullptr;       // [rows16][fp] squared-ReLU activations (f32)
    float* pmax = nullptr;       // [rows16][heads] each head's largest magnitude in gatedf
    float* out = nullptr;        // [cap][vocab] logits or probabilities
    uint32_t* slots = nullptr;   // [cap] slots of the current step (validated copy)
    uint32_t* d_slots = nullptr; // [3 cap] H2D target of the synchronous entry points: n slots, n tokens,
                                 // then n next symbols or decoder targets (the CDF readers)
    uint32_t* h_slots = nullptr; // [3 cap] pinned staging of the same
    // Pinned staging of the outputs handed back to host memory (up to one round of
    // out_stage_bytes), with one completion event per chunk of a round (at most four).
    unsigned char* h_out = nullptr;
    size_t out_stage_bytes = 0;
    hipEvent_t out_ev[32] = {};
    uint8_t* seen = nullptr;     // host duplicate check, cap bytes
    // Queued calls (forward_batch_cdf_sym_submit / _wait): at most kQueued in flight, each
    // with its own inputs (3 cap u32: slots, tokens, next symbols; pinned and on the
    // device), its results (3 cap u32, pinned) and its completion event.
    static constexpr uint32_t kQueued = 2;
    struct Queued {
        uint32_t* h_in = nullptr;
        uint32_t* d_in = nullptr;
        uint32_t* h_res = nullptr;
        hipEvent_t done = nullptr;
        uint64_t ticket = 0;   // 0: free
        uint32_t n = 0;
    };
    Queued queued[kQueued];
};

// Kernel classes a caller can time with HIP events (see Probe).
enum KernelClass : uint32_t {
    KC_NONE = 0, KC_EMBED = 1, KC_MIX_IN = 2, KC_SCAN = 3, KC_MIX_OUT = 4, KC_HEAD = 5, KC_SOFTMAX = 6,
    // RWKV-7: LayerNorm + token shift, matrix-core projections, WKV-7 (with GroupNorm, bonus, gate)
    KC_SHIFT = 7, KC_PROJ = 8, KC_WKV = 9,
    // the persistent step kernel (every layer of a Mamba step in one launch)
    KC_FLOW = 10,
    KC_NORM = 11, KC_XPROJ = 12,   // the reference-order tier's norms and x_proj
    KC_COUNT = 13
};

// Measurement hook: while cls != KC_NONE, every launch of that class records its dispatch
// start and stop into two events taken in order from ev[0..cap) (ev is caller-owned);
// `used` counts them.  Probed steps run as direct launches, not as the replayed graph.
// With `only`, a probed step launches just that class's kernels between one event pair.
struct Probe {
    uint32_t cls = KC_NONE;
    bool only = false;   // launch only this class, back to back, between one event pair
    hipEvent_t* ev = nullptr;
    uint32_t cap = 0, used = 0;
};

// RWKV-7 (src/infrastructure/rwkv7/model.rs:14-141).
struct RDims {
    uint32_t vocab = 0, d = 0, h = 0, n = 0, nl = 0, f = 0;
    uint32_t lora[4] = {0, 0, 0, 0};   // ranks of the decay (w), a, g and v LoRAs
    uint32_t g1k = 0;
};

enum { kLoraW = 0, kLoraA = 1, kLoraG = 2, kLoraV = 3 };

// A LoRA matrix for the element-wise-exact kernels of the RWKV-7 W8A8 tier: f32, laid out
// [cols / 8][rows8][8] (rows8 = rows rounded up to 8, zero rows past `rows`; cols a
// multiple of 8), so the eight lanes that own the eight column residues of one row read 32
// contiguous bytes and the wave's eight rows 256.
struct LMat {
    int rows = 0, cols = 0, rows8 = 0;
    float* w = nullptr;
};

struct RLayer {
    float *ln1_w = nullptr, *ln1_b = nullptr, *ln2_w = nullptr, *ln2_b = nullptr;
    float* mix[6] = {};               // x_r, x_w, x_k, x_v, x_a, x_g
    float *w0 = nullptr, *a0 = nullptr, *v0 = nullptr, *k_k = nullptr, *k_a = nullptr, *r_k = nullptr;
    float *ln_x_w = nullptr, *ln_x_b = nullptr, *ffn_x_k = nullptr;
    TMat r, k, v, o;                  // [d][d]
    TMat l1[4];                       // first LoRA stages [rank][d] (F32): w1, a1, g1, v1
    TMat l2[4];                       // second LoRA stages [d][rank] (F32): w2, a2, g2, v2
    TMat fk, fv;                      // [d_ffn][d], [d][d_ffn]
    LMat x1[4], x2[4];                // the LoRA stages of the W8A8 and reference-order tiers (l1/l2 stay empty there)
    RowMat e_r, e_k, e_v, e_o, e_fk, e_fv;   // the reference-order tier's projections (the TMats stay empty there)
};

struct RwkvView {
    const RDims* dims;
    const RLayer* layers;
    const TMat* emb;       // [vocab][d] F32, already through ln0
    const TMat* head;      // [vocab][d]
    const float* ln_out_w;
    const float* ln_out_b;
    bool a8;               // the W8A8 tier: int8 activations, element-wise exact
    bool exact;            // the reference-order tier: F32 projections in the reference GEMV's order
    const RowMat* e_head;  // its head [vocab][d]
};

// Scratch and state sizes of an RWKV-7 pool of `cap` streams (elements).  The limb
// buffers serve the matrix-core tiers, the a8 ones the W8A8 and reference-order tiers (the
// other set is empty); the reference-order tier keeps six f32 token-shift outputs in mixf.
struct RwkvSizes {
    size_t state_d, wkv, mixl, loral, lora_off[4], gatedl, actl;
    int ks_d, ks_f, ks_lora[4];
    // W8A8: padded row lengths of the activations, their rows (cap rounded up to 16), the
    // first LoRA stages' offsets in one [cap][lora_sum] row, and the buffer sizes
    size_t dp, fp, rows16, lh_off[4], lora_sum, mixf, lorah, aq, as, gatedf, actf, pmax;
};
// int8 activation vectors of the W8A8 tier in Pool::aq, [rows16][dp] each (kAqAct, the last:
// [rows16][fp]), with one scale per stream in Pool::as.
enum { kAqR = 0, kAqK = 1, kAqV = 2, kAqFfn = 3, kAqHead = 4, kAqAct = 5, kAqVecs = 6 };
RwkvSizes rwkv_sizes(const RDims& d, uint32_t cap, bool a8, bool exact = false);

struct ModelView {
    const Dims* dims;
    const DLayer* layers;   // host array of nl layers
    const TMat* emb;        // the embedding (tiled like a projection)
    const TMat* head;       // emb when tied
    const float* norm_f_w;
    const float* norm_f_b;
    bool exact_scan;        // scan decay factors by the portable exp (else the hardware exp2)
};

// One step's inputs.  slots/tokens/out are device pointers; `check` validates slots
// and tokens on the device into *err (bit 0: out of range, bit 1: duplicate slot).
// A step may run as several parts (sub-batches of whole 16-stream groups): a part covers
// batch rows [b0, b0 + n) of the step's n_all rows; slots, tokens and out always point at
// row 0 of the whole step, and the device check of every part covers all n_all slots.
struct StepIO {
    uint32_t n;
    const uint32_t* slots;
    const uint32_t* tokens;
    float* out;
    bool probs;
    bool check;
    uint32_t* err;
    uint32_t b0 = 0;
    uint32_t n_all = 0;   // 0: n (one part)
};

// A linear sequence of kernel launches that is either issued directly on a stream or
// recorded once as a hipGraph and replayed.
struct Launch;

// The persistent step kernel's launch on this device: grid (0: it does not run here) and
// the device's XCDs, as XCC_ID -> index 0 .. nx - 1 (0xff where no workgroup was seen).
struct FlowShape {
    uint32_t grid = 0, nx = 0;
    uint32_t fixed = 0;   // 1: static task assignment (see k_flow)
    uint8_t xmap[16] = {};
};

// Builds the launch list of one step of a model; io_i / head_i / sm_i name the launches
// whose arguments carry the caller's pointers (embedding, head, softmax; -1 if absent).
struct StepSource {
    virtual ~StepSource() = default;
    virtual void build(Pool& p, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i,
                       int& sm_i) const = 0;
    // Whether build() accepts a part (io.b0 > 0 or io.n < io.n_all) of a step.
    virtual bool splittable() const { return false; }
    // The persistent step kernel (all layers in one cooperative launch), where the source
    // has one for steps of n streams: flow_bytes() > 0 is the size of its device
    // arguments (per-layer table, phase counters, task tickets), flow_init() writes them
    // into `dev` once per pool and n and returns the launch shape (grid 0: the kernel
    // cannot run on this device; the step then takes build()), and build_flow() makes the
    // step's launch list around it.
    virtual size_t flow_bytes(const Pool&, uint32_t) const { return 0; }
    virtual hipError_t flow_init(Pool&, uint32_t, void*, FlowShape* shape, hipStream_t) const {
        *shape = FlowShape{};
        return hipSuccess;
    }
    virtual void build_flow(Pool&, const StepIO&, void*, const FlowShape&, std::vector<Launch>&) const {}
};

struct MambaStep final : StepSource {
    ModelView m;
    explicit MambaStep(const ModelView& v) : m(v) {}
    void build(Pool& p, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i, int& sm_i) const override;
    bool splittable() const override { return true; }
    size_t flow_bytes(const Pool& p, uint32_t n) const override;
    hipError_t flow_init(Pool& p, uint32_t n, void* dev, FlowShape* shape, hipStream_t st) const override;
    void build_flow(Pool& p, const StepIO& io, void* dev, const FlowShape& shape, std::vector<Launch>& out) const override;
};

// The Mamba step on the wavefront-GEMV kernels (weights in GMat layout).
struct GemvView {
    const Dims* dims;
    const DLayer* layers;
    const GMat* emb;        // the embedding in GEMV layout
    const GMat* head;       // emb when tied
    const float* norm_f_w;
    bool exact_scan;
};

struct GemvStep final : StepSource {
    GemvView m;
    explicit GemvStep(const GemvView& v) : m(v) {}
    void build(Pool& p, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i, int& sm_i) const override;
};

// GEMV layout parameters of a K-column matrix: false if K is not a multiple of 16 or no
// chunks-per-lane count up to 8 divides the lanes evenly.
bool gemv_shape(int cols, int& rpi, int& cpl);

struct ExactView {
    const Dims* dims;
    const DLayer* layers;
    const RowMat* emb;
    const RowMat* head;     // emb when tied
    const float* norm_f_w;
    const float* norm_f_b;
    bool fma;               // numeric contract 2 (fma-v1) instead of 1
};

// The reference-order tier (weight profile bit 6; bit 7 for numeric contract 2): every
// projection in the reference GEMV's own order, sequential norms, the portable exp in the
// scan, one part per step.
struct ExactStep final : StepSource {
    ExactView m;
    explicit ExactStep(const ExactView& v) : m(v) {}
    void build(Pool& p, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i, int& sm_i) const override;
};

// One F32 projection of the reference-order tier in numeric contract 1 (exact_step.hip),
// for the RWKV-7 step: row r of stream b is the reference's dot_avx2_order of W's row r and
// the stream's input row act + b * w.cols, then stored at out[b * ostride + r] (EXACT_STORE),
// added to it (EXACT_RESID), or stored through the squared ReLU (EXACT_RELU2).
enum ExactEpi : int { EXACT_STORE = 0, EXACT_RESID = 2, EXACT_RELU2 = 3 };
Launch exact_gemv_launch(const RowMat& w, const float* act, uint32_t n, float* out, uint32_t ostride, int epi,
                         uint32_t cls);
// Three such products of one shape in one launch (EXACT_STORE), product k's outputs from
// out + out_off[k] (out_off ascending).
Launch exact_gemv3_launch(const RowMat* const (&w)[3], const float* const (&act)[3], uint32_t n, float* out,
                          const uint32_t (&out_off)[3], uint32_t ostride, uint32_t cls);

struct RwkvStep final : StepSource {
    RwkvView m;
    explicit RwkvStep(const RwkvView& v) : m(v) {}
    void build(Pool& p, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i, int& sm_i) const override;
    // The matrix-core tier runs a step as parts; the W8A8 and reference-order tiers in one.
    bool splittable() const override { return !m.exact && !m.a8; }
    // The W8A8 tier's step and the reference-order tier's (rwkv_a8.hip).
    void build_a8(Pool& p, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i, int& sm_i) const;
    void build_ref(Pool& p, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i, int& sm_i) const;
};

// Most parts a step is split into: one per hardware queue a process gets by default.
constexpr uint32_t kMaxParts = 4;
// Streams per part at least: below it the parts' kernels are short enough that running
// two of them at once loses more (each wave slower, the XCD-aware layouts interleaved
// with another kernel's) than it overlaps.  Measured on Mamba-130M int8, parts per step:
// 128 streams 702 / 645 / 687 / 1050 us for 1 / 2 / 3 / 4 parts, 1024 streams 2980 /
// 2732 / - / 3245 us, 32 streams 379 / 456 us for 1 / 2; one / two parts at 96 streams
// 653 / 571 us, at 112 684 / 589 us, at 80 493 / 543 us.
constexpr uint32_t kMinPartStreams = 48;
// Parts per step by default (REDUKT_GPU_SPLIT overrides).
constexpr uint32_t kDefaultSplit = 2;
// Smallest step that runs the persistent step kernel by default (REDUKT_GPU_FLOW
// overrides; 0 = never).
constexpr uint32_t kDefaultFlowFrom = 0;
constexpr uint32_t kDefaultSkew = 1;

class StepRunner {
public:
    StepRunner() = default;
    StepRunner(const StepRunner&) = delete;
    StepRunner& operator=(const StepRunner&) = delete;
    // Releases this runner's graphs, streams and events, then takes over o's.
    StepRunner& operator=(StepRunner&& o) noexcept;
    ~StepRunner();
    // Destroys every graph, stream and event of the runner.
    void release();
    // Issue one step.  Builds (or reuses) the graphs of this shape unless a probe is
    // active, in which case the step is launched directly (as one part) with events around
    // the probed class.  A splittable step of n streams runs as up to split() parts of whole
    // 16-stream groups, part k on its own stream (part 0 on st), forked from and joined back
    // into st by events, so the parts' kernels overlap.  Returns hipSuccess or the first error.
    hipError_t run(const StepSource& src, Pool& p, const StepIO& io, hipStream_t st, Probe* probe);
    // One step as direct launches on st, in one part: no graph is captured and no stream,
    // event or device memory is created.
    hipError_t run_direct(const StepSource& src, Pool& p, const StepIO& io, hipStream_t st);
    void clear();
    // Parts per step (1 .. kMaxParts) and the fewest streams a part may have; the streams
    // and events are created on first use.
    void set_split(uint32_t k, uint32_t min_part = kMinPartStreams) {
        split_ = k < 1 ? 1 : (k > kMaxParts ? kMaxParts : k);
        min_part_ = min_part < 1 ? 1 : min_part;
    }
    uint32_t split() const { return split_; }
    // Steps of at least `from` streams (0: none) whose source has a persistent step kernel
    // run it (direct launches, one part) instead of the per-layer graphs.
    void set_flow(uint32_t from) { flow_from_ = from; }
    // A split step issues the first `k` launches of each part but the last before the next
    // part starts, so consecutive parts run that many kernels apart (0: all parts start
    // together).
    void set_skew(uint32_t k) { skew_ = k; }
    // Rows [b0, b0 + n) of each part of a step of n streams split at most k ways.
    static uint32_t parts_of(uint32_t n, uint32_t k, uint32_t* b0, uint32_t* cnt);

private:
    struct Part {
        uint32_t b0 = 0, n = 0;
        bool updatable = false;
        hipGraph_t g = nullptr;
        hipGraphExec_t exec = nullptr;
        hipGraphNode_t io_node = nullptr, head_node = nullptr, softmax_node = nullptr;
        std::vector<Launch>* launches = nullptr;  // argument storage, alive as long as the graph
        int io_i = -1, head_i = -1, sm_i = -1;
        uint32_t lead = 0;   // leading launches issued directly, before the next part starts (the graph holds the rest)
    };
    struct Graph {
        uint32_t n = 0, split = 1;
        bool probs = false, check = false;
        const Pool* pool = nullptr;
        // Caller pointers the graphs were last launched with; when every part's nodes that
        // carry them were found (`updatable`), other pointers are set in place.
        const uint32_t* tokens = nullptr;
        const uint32_t* slots = nullptr;
        const float* out = nullptr;
        const uint32_t* err = nullptr;
        uint32_t nparts = 0;
        Part parts[kMaxParts];
        uint64_t last_use = 0;
        bool updatable() const;
    };
    // The persistent step kernel's device arguments for one pool and batch size.
    struct FlowPlan {
        const Pool* pool = nullptr;
        uint32_t n = 0;
        FlowShape shape;            // grid 0: the kernel cannot run here, use the graphs
        void* dev = nullptr;
        uint64_t last_use = 0;
    };
    hipError_t capture(const std::vector<Launch>& seq, uint32_t first, hipStream_t st, Part& pt);
    hipError_t streams_ready(hipStream_t st, uint32_t parts);
    hipError_t flow_plan(const StepSource& src, Pool& p, uint32_t n, size_t bytes, hipStream_t st, FlowPlan*& out);
    void destroy(Graph& g);
    std::vector<Graph> graphs_;
    std::vector<FlowPlan> plans_;
    uint32_t flow_from_ = 0;
    uint64_t clock_ = 0;
    uint32_t split_ = 1, min_part_ = kMinPartStreams;
    uint32_t skew_ = 0;
    hipStream_t aux_[kMaxParts] = {};        // aux_[k] runs part k (k >= 1)
    hipEvent_t fork_[kMaxParts] = {};        // recorded on part k's stream after its lead; part k + 1 waits for it
    hipEvent_t join_[kMaxParts] = {};
    std::vector<Launch> direct_;             // run_direct's launch list (host storage, reused)
};

// Zero the state of the n slots listed in d_slots (device).  Uses no memset, so it is
// safe under stream capture.
hipError_t enqueue_reset(const Dims& dims, Pool& pool, const uint32_t* d_slots, uint32_t n, hipStream_t stream);
hipError_t enqueue_reset_rwkv(const RDims& dims, Pool& pool, const uint32_t* d_slots, uint32_t n, hipStream_t stream);

// Scratch sizes of a pool of `cap` streams.
size_t xpart_floats(const Dims& d, uint32_t cap);
size_t glimb_elems(const Dims& d, uint32_t cap);
size_t xw_elems(const Dims& d, uint32_t cap);
size_t ssp_floats(const Dims& d, uint32_t cap);

}  // namespace rdk
