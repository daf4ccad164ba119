/* Lockstep compress / decompress driver of redukt's host over a GPU backend plugin.
 *
 * The host side of src/application/lockstep.rs (run_lockstep, R-100) and of the plugin
 * backbone it drives (src/infrastructure/plugin_backend/model.rs:32-103, 357-452):
 *
 *   - the plugin library is loaded with dlopen and bound by symbol name, as the reference
 *     loader does (plugin_backend/loader.rs:116-153); v1 symbols are required, the v2
 *     batch symbols are required for more than one slot;
 *   - N slots advance one token per step.  Phase A (host thread pool, one unit per active
 *     stream): build the stream's CDF from the logits of its previous forward (the first
 *     token uses the uniform CDF) and code its next token.  Finished streams then leave.
 *     Phase B: one forward_batch for every stream still running, after each stream's
 *     periodic-reset tick;
 *   - continuous batching: a freed slot takes the next file at the start of a step, after
 *     a reset of its state;
 *   - identity: a file's coded bytes do not depend on the slot count, the slot it lands
 *     in, its batch neighbours or the thread count, and equal the single-stream (v1)
 *     path's bytes (tests/roundtrip.rs:681-736).
 *
 * Scope: the token stream is coded with CDFs built straight from the backbone's logits
 * (the shape of the reference's own codec test, src/application/codec.rs:3255-3290).
 * The reference CLI additionally mixes its CPU context models into the logits before
 * the CDF; that mixing is not part of this library, so its archives are not decodable
 * by the reference CLI and vice versa.
 *
 * The plugin is a process-global singleton: one driver at a time per process, and no
 * other user of the same plugin library while it is open.
 */
#ifndef REDUKT_LOCKSTEP_H
#define REDUKT_LOCKSTEP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct redukt_lockstep redukt_lockstep;

typedef enum {
    REDUKT_LOCKSTEP_OK = 0,
    REDUKT_LOCKSTEP_INVALID_ARG = 1,
    REDUKT_LOCKSTEP_PLUGIN_LOAD = 2,     /* dlopen or a required symbol failed */
    REDUKT_LOCKSTEP_PLUGIN_INIT = 3,     /* init / init_ex / batch_init returned an error */
    REDUKT_LOCKSTEP_FORWARD = 4,         /* forward / forward_batch / batch_reset failed */
    REDUKT_LOCKSTEP_CODER = 5,           /* a file's coder failed (see its status) */
    REDUKT_LOCKSTEP_BUFFER_TOO_SMALL = 6,
    REDUKT_LOCKSTEP_NEEDS_V2 = 7,        /* more than one slot on a v1-only plugin */
} redukt_lockstep_status;

typedef struct {
    uint64_t steps;        /* lockstep steps (Phase A + B rounds) */
    uint64_t tokens;       /* tokens coded */
    uint64_t files;        /* files finished */
    double secs;           /* wall time of the whole run */
    double code_secs;      /* Phase A: CDF construction + coding */
    double forward_secs;   /* Phase B: resets + forward_batch */
} redukt_lockstep_stats;

/* Opens plugin_path, initialises it on weights_path (a .rbin file, or a directory that
 * holds model.rbin) and prepares `slots` streams.  profile < 0 uses the plugin's plain
 * init (its default profile); profile >= 0 calls the optional redukt_backend_init_ex.
 * slots = 0 selects the single-stream path: the plugin's v1 global state, one file at a
 * time (the reference's `compress --input`).  threads = 0 uses every host thread for
 * Phase A.  On failure *out is NULL and the status says which step failed. */
int32_t redukt_lockstep_open(const char* plugin_path, const char* weights_path, int32_t device_id,
                             int32_t profile, uint32_t slots, uint32_t threads, redukt_lockstep** out);
/* Frees the plugin (redukt_backend_free) and unloads it. */
void redukt_lockstep_close(redukt_lockstep* ls);
uint32_t redukt_lockstep_vocab(const redukt_lockstep* ls);
/* The plugin's BackendInfo.name (NUL-terminated, at most 63 characters). */
const char* redukt_lockstep_backend_name(const redukt_lockstep* ls);

/* on = 1: Phase B takes each stream's CDF from the plugin's optional
 * redukt_backend_forward_batch_cdf (computed on the device, bit for bit the host CDF), so
 * Phase A only codes; on = 0: Phase B takes logits and Phase A builds the CDFs on the host.
 * open() turns it on for the lockstep path when the plugin exports forward_batch_cdf.  The bytes
 * are the same either way.  INVALID_ARG when the plugin does not export forward_batch_cdf
 * or the driver runs the single-stream path (slots = 0). */
int32_t redukt_lockstep_set_device_cdf(redukt_lockstep* ls, int32_t on);
/* 1 when Phase B takes CDFs from the plugin. */
int32_t redukt_lockstep_device_cdf(const redukt_lockstep* ls);

/* Upper bound of a coded stream of n tokens: every symbol costs at most 25 bits (a
 * frequency of 1 in 2^24 plus the range truncation), plus the 5-byte flush. */
uint64_t redukt_lockstep_stream_bound(uint64_t n_tokens);

/* Codes files[i] = tokens[i][0 .. n_tokens[i]) (every token < vocab, n_tokens[i] >= 1).
 * The state is zeroed every reset_every forwards (0 = never; the reference's default for
 * the Mamba family is 4096).  Coded stream i goes to out[i] (capacity cap[i]);
 * out_len[i] receives its length (the needed length when it did not fit).  status, if
 * not NULL, receives one redukt_codec_status per file.  Returns OK when every file
 * succeeded, else the first failure.  When the backbone fails mid-run (FORWARD), every
 * file still in flight and every file not yet admitted reports REDUKT_CODEC_INCOMPLETE
 * with out_len 0; files finished before the failure keep their status and bytes. */
int32_t redukt_lockstep_compress(redukt_lockstep* ls, uint32_t n_files, const uint32_t* const* tokens,
                                 const uint64_t* n_tokens, uint64_t reset_every, uint8_t* const* out,
                                 const uint64_t* cap, uint64_t* out_len, int32_t* status,
                                 redukt_lockstep_stats* stats);

/* Restores n_tokens[i] tokens of each coded stream into tokens_out[i]; reset_every must
 * be the value the streams were coded with.  status as for compress (a symbol >= vocab
 * reports SYMBOL_OUT_OF_RANGE and ends that file). */
int32_t redukt_lockstep_decompress(redukt_lockstep* ls, uint32_t n_files, const uint8_t* const* streams,
                                   const uint64_t* stream_len, const uint64_t* n_tokens, uint64_t reset_every,
                                   uint32_t* const* tokens_out, int32_t* status, redukt_lockstep_stats* stats);

#ifdef __cplusplus
}
#endif
#endif /* REDUKT_LOCKSTEP_H */
