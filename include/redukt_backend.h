/* redukt_backend.h — C ABI of libredukt_gpu.so, the MI355X (gfx950) backbone backend.
 *
 * The library is a drop-in replacement for redukt's GPU plugin.  The host loads it
 * with dlopen from next to its executable (src/infrastructure/plugin_backend/loader.rs:116-153)
 * and resolves the symbols below by name.  v1 and v2 are exactly the reference
 * contract; v3 adds optional symbols the unchanged host never looks up.
 *
 * Contract summary (docs/api/PLUGIN-FFI-V2.md:7-108):
 *   - process-global singleton, single-threaded, not reentrant;
 *   - all calls synchronous: outputs are complete when a call returns;
 *   - the caller owns every pointer argument for the duration of the call only;
 *   - a stream's logits are bit-identical whether it runs through v1 or inside any
 *     v2 batch, at any batch position and slot, and run after run.
 */
#ifndef REDUKT_BACKEND_H
#define REDUKT_BACKEND_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Result codes — src/domain/backend_ffi.rs:27-41.  v1 entry points return the enum
 * (int-sized), v2/v3 entry points return int32_t. */
typedef enum {
    BACKEND_OK = 0,
    BACKEND_INIT_FAILED = 1,
    BACKEND_FORWARD_FAILED = 2,
    BACKEND_VERSION_MISMATCH = 3,
    BACKEND_WEIGHTS_NOT_FOUND = 4,
    BACKEND_INVALID_ARGUMENT = 5,
} BackendResult;

#define BACKEND_FFI_VERSION 1   /* BackendInfo.ffi_version, backend_ffi.rs:16 */
#define BACKEND_ABI_VERSION 3   /* redukt_backend_abi_version(): v2 batch + v3 extensions */
#define BACKEND_NAME_MAX 64
#define BACKEND_MAX_STREAMS 4096u

/* 76 bytes, backend_ffi.rs:63-72. */
typedef struct {
    uint32_t ffi_version;
    uint32_t vocab_size;
    uint32_t hidden_dim;
    uint8_t name[BACKEND_NAME_MAX];
} BackendInfo;

/* ---------------- v1 (backend_ffi.rs:91-114) ---------------- */

/* Replaces BackendInitFn (backend_ffi.rs:91-95).  weights_path: NUL-terminated path to
 * a .rbin file, or a directory holding model.rbin.  device_id < 0 means 0.  Re-init
 * frees everything first.  Bad or missing weights -> WEIGHTS_NOT_FOUND; device
 * failure -> INIT_FAILED.  The weight profile (F32 / Q8) is taken from the
 * REDUKT_GPU_PROFILE environment variable ("f32" default, "q8", "q8row", "q8row-all")
 * or chosen explicitly with redukt_backend_init_ex. */
BackendResult redukt_backend_init(const uint8_t* weights_path, int32_t device_id, BackendInfo* info_out);

/* Replaces BackendForwardFn (backend_ffi.rs:102-106): one token on the private v1
 * state; any error (vocab mismatch included) -> FORWARD_FAILED. */
BackendResult redukt_backend_forward(uint32_t token, float* out_logits, uint32_t vocab_size);

/* Replaces BackendResetFn (backend_ffi.rs:110): zero the v1 state. */
void redukt_backend_reset_state(void);

/* Replaces BackendFreeFn (backend_ffi.rs:114): release everything. */
void redukt_backend_free(void);

/* ---------------- v2 (backend_ffi.rs:136-177) ---------------- */

/* Replaces BackendAbiVersionFn (backend_ffi.rs:137); returns BACKEND_ABI_VERSION. */
uint32_t redukt_backend_abi_version(void);

/* Replaces BackendBatchInitFn (backend_ffi.rs:142): free the old pool, allocate
 * max_streams zeroed slots; 0 only frees.  INIT_FAILED without a model or on OOM,
 * INVALID_ARGUMENT above BACKEND_MAX_STREAMS. */
int32_t redukt_backend_batch_init(uint32_t max_streams);

/* Replaces BackendBatchResetFn (backend_ffi.rs:146): zero the listed slots
 * (slots == NULL: every slot).  INIT_FAILED without a pool, INVALID_ARGUMENT for a
 * slot >= max_streams (nothing is reset then). */
int32_t redukt_backend_batch_reset(const uint32_t* slots, uint32_t n_slots);

/* Replaces BackendForwardBatchFn (backend_ffi.rs:156-162): advance each listed slot by
 * one token and write row b of out_logits (n_streams * vocab_size f32, row-major).
 * INIT_FAILED without a pool; INVALID_ARGUMENT (vocab mismatch, n > pool, slot >= pool,
 * duplicate slot, token >= vocab, null pointer) launches nothing and changes no
 * state.  n_streams == 0 is a no-op. */
int32_t redukt_backend_forward_batch(uint32_t n_streams, const uint32_t* slots, const uint32_t* tokens,
                                     float* out_logits, uint32_t vocab_size);

/* ---------------- v3 extensions (optional; no counterpart in the reference ABI) ----
 * The reference host resolves only the eight symbols above; these are looked up by
 * hosts that know abi_version() >= 3, the way v2 was added (PLUGIN-FFI-V2.md:7-25). */

/* Weight profiles (bit field): low two bits 0 = F32, 1 = Q8 with one scale per 64
 * columns (the reference's Q8 profile, src/infrastructure/mamba/model.rs:56),
 * 2 = Q8 with one scale per output row; bit 2 = also quantize x_proj and dt_proj.
 * Quantization follows Q8wMatrix::quantize (src/domain/gemv.rs:256-273) at load. */
#define BACKEND_PROFILE_F32 0u
#define BACKEND_PROFILE_Q8_G64 1u
#define BACKEND_PROFILE_Q8_ROW 2u
#define BACKEND_PROFILE_Q8_SMALL 4u
/* Profile bit 3: the Mamba scan's decay factors exp(-dt*A) by the reference's portable
 * exp (bit-identical element-wise scan) instead of the hardware exp2 (about 1e-7
 * relative; the default).  REDUKT_GPU_EXACT_SCAN=1 sets it for redukt_backend_init. */
#define BACKEND_PROFILE_EXACT_SCAN 8u
/* Profile bit 4: the Mamba projections on wavefront-GEMV kernels (f32 dot products on the
 * vector ALUs, weights streamed in a GEMV layout) instead of the matrix cores: the
 * small-batch tier.  The tier is fixed at init for every batch size, so a stream's bits do
 * not depend on n within it (they differ between tiers, like between builds).  F32 or
 * per-row int8 weights (low bits 0 or 2), RMSNorm Mamba models with d_conv 4 and
 * d_model / d_inner in {64, 96, 128, 192, 256, 384, 768, 1024, 1536, 3072}; INIT_FAILED
 * otherwise. */
#define BACKEND_PROFILE_GEMV 16u
/* Profile bit 5: RWKV-7 in the reference's own int8 arithmetic, W8A8 (Q8Tensor and
 * q8_mat_vec_mul_into, src/domain/tensor.rs:105-143, 1791-1866): every per-row int8
 * projection quantizes its input vector to int8 with one scale, sums exact int32 products
 * on the matrix cores and rescales once per row; the rest of the step keeps the reference's
 * operation order, its sequential sums included, so the logits equal the CPU path's bit for
 * bit.  Needs per-row weights (low bits 2) and LoRA ranks in multiples of 8; INIT_FAILED for
 * Mamba models or another profile. */
#define BACKEND_PROFILE_W8A8 32u
/* Profile bit 6: Mamba in the reference CPU path's own arithmetic, the reference-order tier.
 * Every projection (in_proj, x_proj, dt_proj, out_proj, head) is the reference GEMV of each
 * output row, f32_rows / q8w_rows (src/domain/gemv.rs:181-194, 459-502): eight accumulators
 * by column residue, the fixed horizontal sum, the sequential tail, Q8 rows folded over
 * their column groups; the norms are the reference's sequential sums
 * (src/domain/tensor.rs:900-908, 1390-1398) and the scan takes the portable exp, so the
 * logits and the recurrent state equal the CPU path's (numeric contract 1, the "Plain"
 * kernel family) bit for bit, for F32, group-64 and per-row int8 weights alike.  On an
 * RWKV-7 model bit 6 alone (F32 weights) runs its step the same way: every projection in
 * mat_vec_mul_into's dot_avx2_order (src/domain/tensor.rs:1602-1693), the element-wise code
 * and the sums of the W8A8 tier; RWKV-7 with another low bit or bit 7 -> INIT_FAILED (its
 * int8 arithmetic is bit 5's).  Slower than the other tiers: its GEMVs are f32 dot products
 * on the vector ALUs, eight lanes per output. */
#define BACKEND_PROFILE_EXACT 64u
/* Profile bit 7: the reference-order tier in numeric contract 2 (fma-v1,
 * src/domain/gemv_fma.rs:1-134): the same orders with every acc + w * x of a projection,
 * and every sum + dot * scale of a Q8 row, one fused multiply-add.  Implies bit 6. */
#define BACKEND_PROFILE_FMA 128u

/* redukt_backend_init with an explicit weight profile (the model file stays F32); a profile
 * with a bit above bit 7 -> INVALID_ARGUMENT. */
int32_t redukt_backend_init_ex(const uint8_t* weights_path, int32_t device_id, uint32_t profile,
                               BackendInfo* info_out);

/* forward_batch that returns the probability vector softmax(logits) per stream
 * instead of the logits, computed on the device in the order of softmax_into
 * (src/domain/tensor.rs:1917-1933).  Same validation and state rules as forward_batch. */
int32_t redukt_backend_forward_batch_probs(uint32_t n_streams, const uint32_t* slots, const uint32_t* tokens,
                                           float* out_probs, uint32_t vocab_size);

/* forward_batch that returns each stream's CDF (vocab + 1 cumulative u32 frequencies,
 * total 2^24) instead of its logits: the host coding path's redukt_cdf_from_logits
 * (codec.rs:785-798, coder.rs:43-81, the f64 exp of fmath.rs:340-430) computed on the
 * device, bit for bit.  cdf_len must be vocab + 1; out_cdf holds n_streams * cdf_len u32.
 * Same validation and state rules as forward_batch.  No reference counterpart: the
 * reference's roadmap names the on-device CDF (docs/ROADMAP.md:2995) without an
 * interface. */
int32_t redukt_backend_forward_batch_cdf(uint32_t n_streams, const uint32_t* slots, const uint32_t* tokens,
                                         uint32_t* out_cdf, uint32_t cdf_len);

/* forward_batch_cdf for a caller that knows each stream's next symbol (compression): the
 * same CDF rows are computed on the device, and only what the range coder reads of each
 * (coder.rs:163-177) comes back: out_bounds[3b .. 3b + 2] = cdf[next_syms[b]],
 * cdf[next_syms[b] + 1] and cdf[vocab_size], the total.  12 bytes per stream instead of
 * 4 (vocab + 1).  vocab_size must be the model's; next_syms[b] < vocab_size.  Same
 * validation and state rules as forward_batch.  No reference counterpart (an extension of
 * the CDF entry point above). */
int32_t redukt_backend_forward_batch_cdf_sym(uint32_t n_streams, const uint32_t* slots, const uint32_t* tokens,
                                             const uint32_t* next_syms, uint32_t* out_bounds, uint32_t vocab_size);

/* forward_batch_cdf for a range decoder that knows each stream's target cumulative
 * frequency (decompression; the target is the decoder's get_freq value for a total of
 * REDUKT_CDF_TOTAL, which every device CDF row sums to): the same CDF rows are computed on
 * the device and searched there as decode_symbol searches them (coder.rs:100-115);
 * out_found[4b .. 4b + 3] = s, cdf[s], cdf[s + 1] and cdf[vocab_size], the total, with s
 * the symbol found (s = vocab_size and both bounds the total when targets[b] >= the
 * total).  16 bytes per stream instead of 4 (vocab + 1).  vocab_size must be the model's.
 * Same validation and state rules as forward_batch.  No reference counterpart (an
 * extension of the CDF entry point above). */
int32_t redukt_backend_forward_batch_cdf_find(uint32_t n_streams, const uint32_t* slots, const uint32_t* tokens,
                                              const uint32_t* targets, uint32_t* out_found, uint32_t vocab_size);

/* forward_batch_cdf_sym in two halves, so that a caller that knows its next inputs
 * (compression) can queue the next step before it has used this one's results: _submit
 * validates and queues the step, the device CDF and the copy of the three values per
 * stream, and returns at once with *ticket naming the call; _wait(ticket) waits for that
 * call and writes out_bounds (3 u32 a stream, n_streams as submitted).  At most two calls
 * are in flight: a third _submit before one of them is waited for is refused.  Calls run in
 * submission order, after and before every other entry point's work, and each sees the
 * recurrent state its predecessors left; batch_init and free wait for the calls in flight
 * and drop them (their tickets are refused afterwards).  Same validation and state rules
 * as forward_batch.  No reference counterpart (an extension of the CDF entry points above). */
int32_t redukt_backend_forward_batch_cdf_sym_submit(uint32_t n_streams, const uint32_t* slots, const uint32_t* tokens,
                                                    const uint32_t* next_syms, uint32_t vocab_size, uint64_t* ticket);
int32_t redukt_backend_forward_batch_cdf_sym_wait(uint64_t ticket, uint32_t* out_bounds, uint32_t n_streams);

/* The device CDF on caller logits: d_logits [rows][n] f32 -> d_cdf [rows][n + 1] u32,
 * both device pointers, stream-ordered on redukt_backend_stream() (the call does not
 * wait).  1 <= n < 2^24.  For tests and for callers that hold logits on the device. */
int32_t redukt_backend_cdf_from_logits_device(const float* d_logits, uint32_t rows, uint32_t n, uint32_t* d_cdf);

/* Stream-ordered step on device-resident inputs: d_slots, d_tokens and d_out are
 * device pointers (n_streams u32, n_streams u32, n_streams*vocab_size f32).  Nothing is
 * copied to or from the host and the call does not wait for the step to finish.
 * Slots and tokens are checked on the device (against every stream of the call): an
 * invalid entry, or a slot an earlier entry already names, sets a sticky error that
 * redukt_backend_device_status() reports and is stepped on a scratch slot of the pool
 * instead of a real one, so it never touches another stream's state and no index leaves
 * the pool; the valid entries (a repeated slot's first entry included) advance as in a
 * valid call.  flags bit 0: write probabilities instead of logits. */
int32_t redukt_backend_forward_batch_device(uint32_t n_streams, const uint32_t* d_slots, const uint32_t* d_tokens,
                                            float* d_out, uint32_t vocab_size, uint32_t flags);

/* Allocation-free variant of redukt_backend_forward_batch_device.  No counterpart in the
 * reference ABI: it is for callers that cannot allocate device memory around a step
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, checks and results as forward_batch_device; Mamba models only.  The
 * per-step scratch (activations, x_proj partials, the validated slot list) comes from a
 * 16 MiB device array the library holds on each device it runs on until the process ends;
 * the recurrent state stays in the batch pool (batch_init).  The step runs as direct
 * kernel launches on the library's stream: no graph, stream, event or device memory is
 * created and no allocating routine is called.  The scratch bounds n_streams (44,736 bytes
 * a stream at Mamba-130M: at most 374 streams); above it INVALID_ARGUMENT, nothing
 * launched.  Every call on a device shares that scratch and clears the part it uses:
 * calls are ordered on the library's stream, so only calls from several threads can
 * overlap, and those race. */
int32_t redukt_backend_forward_batch_device_noalloc(uint32_t n_streams, const uint32_t* d_slots,
                                                    const uint32_t* d_tokens, float* d_out, uint32_t vocab_size,
                                                    uint32_t flags);

/* Wait for queued work; returns OK, INVALID_ARGUMENT if a device-side check of
 * forward_batch_device failed since the last call, or FORWARD_FAILED if the persistent
 * step kernel gave up waiting for a phase or ran on an XCD it was not planned for (its
 * outputs are then not to be used); the flag is cleared either way. */
int32_t redukt_backend_device_status(void);

/* The hipStream_t every kernel of the library is launched on, as an opaque pointer,
 * so a caller can time the step with events on that stream.  NULL before init. */
void* redukt_backend_stream(void);

/* Measurement hook.  While kernel_class != 0, every launch of that kernel class fills
 * two hipEvent_t taken in order from events[0..n_events) (caller owned, alive while
 * probing); recording stops when they run out.  Classes: 1 embed,
 * 2 mix_in (norm + in_proj + conv + x_proj partials), 3 scan (dt_proj + selective scan +
 * gate), 4 mix_out (out_proj + residual), 5 head (final norm + LM head), 6 softmax;
 * RWKV-7: 7 shift (LayerNorm + token shift), 8 proj (matrix-core projections), 9 wkv (WKV-7
 * with GroupNorm, bonus and gate), plus 1, 5, 6.  Class 10 is the persistent step kernel
 * (every layer of a Mamba step in one cooperative launch, where REDUKT_GPU_FLOW enables it):
 * its launch is bracketed by an event pair recorded on the library's stream, and
 * REDUKT_PROBE_CLASS_ONLY does not apply to it (the step runs whole).
 * Probed launches record their own dispatch start and stop (hipExtLaunchKernel), and
 * probed steps are launched kernel by kernel instead of from the step's hipGraph.
 * With REDUKT_PROBE_CLASS_ONLY or'ed into kernel_class, a probed step launches only the
 * kernels of that class, back to back, between one pair of events: the other kernels
 * of the step do not run (timing only; the recurrent state does not advance as in a
 * real step).  kernel_class 0 switches the probe off.  Returns OK or INVALID_ARGUMENT. */
#define REDUKT_PROBE_CLASS_ONLY 0x100u
int32_t redukt_backend_probe_kernel(uint32_t kernel_class, void** events, uint32_t n_events);

/* Number of events the current probe has recorded. */
uint32_t redukt_backend_probe_used(void);

/* Copy the recurrent state of one batch-pool slot and layer to host memory:
 * conv (d_inner*(d_conv-1) f32), ssm (d_inner*d_state f32); either may be NULL. */
int32_t redukt_backend_get_state(uint32_t slot, uint32_t layer, float* conv_out, float* ssm_out);

/* RWKV-7 models (weights in the RWKV-7 container: .rbin header with version 3, model 2).
 * The state of one batch-pool slot and layer (Rwkv7State, src/infrastructure/rwkv7/
 * model.rs:115-141): the two token-shift inputs (d_model f32 each) and the WKV-7 matrices
 * [n_head][head_size][head_size] (row i, column j); any pointer may be NULL.
 * INVALID_ARGUMENT for a Mamba model. */
int32_t redukt_backend_get_rwkv_state(uint32_t slot, uint32_t layer, float* x_att, float* wkv, float* x_ffn);

/* Test hook, no counterpart in the reference: evaluates one of the portable element-wise
 * functions on the device for n host inputs (y[i] = f(x[i])), so that tests can compare
 * its bits with the CPU path's.  fn: 0 exp (tensor.rs:765-794), 1 lane exp (NaN -> lower
 * clamp, :877-879), 2 ln (:799-837), 3 softplus (:859-861), 4 lane sigmoid (:883-885),
 * 5 sigmoid 1 / (1 + exp(-x)).  Needs no model; allocates and synchronizes. */
#define REDUKT_MATH_FN_COUNT 6u
int32_t redukt_backend_eval_math(uint32_t fn, const float* x, float* y, uint32_t n);

/* Measurement hook, no counterpart in the reference: copies `bytes` from device memory src
 * to device memory dst on the library's stream (the default stream before init) with a
 * kernel whose lanes move 4 bytes per load and store (mode bit 1 clear) or 16 (set), with
 * the default cache policy (mode bit 0 clear) or the streaming one the recurrent state uses
 * (set).  Hardware byte counters (FETCH_SIZE, WRITE_SIZE) read on such a copy of known
 * size give the scale for kernels whose traffic has that shape.  Stream-ordered: returns
 * once the copy is queued.  INVALID_ARGUMENT for a mode above 3, bytes not a multiple of
 * 16 or not below 2^31, or a null pointer with bytes > 0. */
int32_t redukt_backend_copy_probe(void* dst, const void* src, uint64_t bytes, uint32_t mode);

#ifdef __cplusplus
}
#endif
#endif
