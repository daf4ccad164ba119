// Lockstep compress / decompress over a GPU backend plugin (src/application/lockstep.rs,
// src/infrastructure/plugin_backend/model.rs).  One driver object owns the loaded plugin,
// one host logits buffer [slots x vocab] that forward_batch fills, and one CDF buffer
// [slots x (vocab + 1)] that Phase A fills row by row on the host thread pool.
#include "redukt_lockstep.h"

#include <dlfcn.h>

#include <chrono>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "coder.h"
#include "host_pool.h"
#include "redukt_backend.h"

namespace {

using Clock = std::chrono::steady_clock;

double since(Clock::time_point t0) { return std::chrono::duration<double>(Clock::now() - t0).count(); }

// Symbols bound by name (plugin_backend/loader.rs:116-153 for v1, the v2 vtable for the
// batch API; init_ex is this backend's optional profile selector).
struct PluginApi {
    void* handle = nullptr;
    BackendResult (*init)(const uint8_t*, int32_t, BackendInfo*) = nullptr;
    BackendResult (*forward)(uint32_t, float*, uint32_t) = nullptr;
    void (*reset_state)() = nullptr;
    void (*free_all)() = nullptr;
    uint32_t (*abi_version)() = nullptr;
    int32_t (*batch_init)(uint32_t) = nullptr;
    int32_t (*batch_reset)(const uint32_t*, uint32_t) = nullptr;
    int32_t (*forward_batch)(uint32_t, const uint32_t*, const uint32_t*, float*, uint32_t) = nullptr;
    int32_t (*init_ex)(const uint8_t*, int32_t, uint32_t, BackendInfo*) = nullptr;
    // optional: forward_batch that hands back each stream's CDF computed on the device
    int32_t (*forward_batch_cdf)(uint32_t, const uint32_t*, const uint32_t*, uint32_t*, uint32_t) = nullptr;
    // optional: the same, handing back only the coder's three values for a known next symbol
    int32_t (*forward_batch_cdf_sym)(uint32_t, const uint32_t*, const uint32_t*, const uint32_t*, uint32_t*,
                                     uint32_t) = nullptr;
    // optional: forward_batch_cdf_sym queued (submit) and collected (wait)
    int32_t (*cdf_sym_submit)(uint32_t, const uint32_t*, const uint32_t*, const uint32_t*, uint32_t,
                              uint64_t*) = nullptr;
    int32_t (*cdf_sym_wait)(uint64_t, uint32_t*, uint32_t) = nullptr;
    // optional: the same, searching each row on the device for the decoder's target
    int32_t (*forward_batch_cdf_find)(uint32_t, const uint32_t*, const uint32_t*, const uint32_t*, uint32_t*,
                                      uint32_t) = nullptr;
    bool v2 = false;

    template <class F>
    void bind(F& fn, const char* name) {
        fn = reinterpret_cast<F>(dlsym(handle, name));
    }

    bool load(const char* path) {
        handle = dlopen(path, RTLD_NOW | RTLD_LOCAL);
        if (!handle) return false;
        bind(init, "redukt_backend_init");
        bind(forward, "redukt_backend_forward");
        bind(reset_state, "redukt_backend_reset_state");
        bind(free_all, "redukt_backend_free");
        if (!init || !forward || !reset_state || !free_all) return false;
        bind(abi_version, "redukt_backend_abi_version");
        bind(batch_init, "redukt_backend_batch_init");
        bind(batch_reset, "redukt_backend_batch_reset");
        bind(forward_batch, "redukt_backend_forward_batch");
        bind(init_ex, "redukt_backend_init_ex");
        bind(forward_batch_cdf, "redukt_backend_forward_batch_cdf");
        bind(forward_batch_cdf_sym, "redukt_backend_forward_batch_cdf_sym");
        bind(forward_batch_cdf_find, "redukt_backend_forward_batch_cdf_find");
        bind(cdf_sym_submit, "redukt_backend_forward_batch_cdf_sym_submit");
        bind(cdf_sym_wait, "redukt_backend_forward_batch_cdf_sym_wait");
        v2 = abi_version && batch_init && batch_reset && forward_batch && abi_version() >= 2;
        return true;
    }
};

enum class Mode { Encode, Decode };

constexpr uint32_t kDeviceCdfFrom = 1;    // slots from which Phase B takes CDFs from the plugin

// A slot's file in flight (lockstep.rs:71-97 without the context-mixing models).
struct Lane {
    int64_t file = -1;  // -1: free
    uint64_t pos = 0;
    uint32_t next_token = 0;
    bool done = false;
    int32_t status = REDUKT_CODEC_OK;
    uint64_t since_reset = 0;  // PluginState::tick schedule
    uint32_t row = 0;          // logits row of this lane's last forward
    int32_t target_status = REDUKT_CODEC_OK;  // the decoder target's status for that forward
    uint64_t code_pos = 0;     // pipelined compression: the position this iteration codes
    uint32_t code_row = 0;     // and its row in the previous forward
    bool leaves = false;       // and whether the file ends with it
    redukt_rc_encoder enc;
    redukt_rc_decoder dec;
};

// The inputs and outputs of one compress or decompress call.
struct Job {
    Mode mode;
    uint32_t n_files;
    const uint64_t* n_tokens;
    uint64_t reset_every;
    // encode
    const uint32_t* const* tokens = nullptr;
    uint8_t* const* out = nullptr;
    const uint64_t* cap = nullptr;
    uint64_t* out_len = nullptr;
    // decode
    const uint8_t* const* streams = nullptr;
    const uint64_t* stream_len = nullptr;
    uint32_t* const* tokens_out = nullptr;
    int32_t* status = nullptr;
};

}  // namespace

struct redukt_lockstep {
    PluginApi api;
    BackendInfo info{};
    uint32_t vocab = 0;
    uint32_t slots = 0;  // 0: the v1 single-stream path
    uint32_t threads = 0;
    // Phase B takes the CDFs from the plugin (forward_batch_cdf, rows in forward order)
    // instead of logits; Phase A then only codes.
    bool device_cdf = false;
    // Compression with device CDFs takes, where the plugin has it, only the three values of
    // each row the coder reads for the lane's next symbol (forward_batch_cdf_sym): 12 bytes
    // a stream cross from the device instead of the whole row.  Decompression likewise
    // sends each lane's decoder target and takes back the symbol found with its bounds
    // (forward_batch_cdf_find, 16 bytes a stream).
    bool sym_cdf = false;
    bool find_cdf = false;
    // Compression on that path queues each step's forward before it codes the previous
    // step's results (forward_batch_cdf_sym_submit / _wait): the device never waits for the
    // host between steps.
    bool pipeline = false;
    std::vector<float> logits;
    std::vector<uint32_t> cdf;
    std::vector<uint32_t> uniform;
    std::vector<uint32_t> bounds;  // [row][3] of the last forward_batch_cdf_sym, [row][4] of _find

    const uint32_t* cdf_row(uint32_t i) const { return cdf.data() + size_t(i) * (vocab + 1); }
    uint32_t* cdf_row(uint32_t i) { return cdf.data() + size_t(i) * (vocab + 1); }
    const float* logits_row(uint32_t r) const { return logits.data() + size_t(r) * vocab; }

    // Phase A for one lane (lockstep.rs:code_step): CDF of the previous forward's logits
    // (uniform for the first token), then code the token at pos.
    void code_step(const Job& job, Lane& l, uint32_t lane_index) {
        const uint32_t* c = uniform.data();
        if (l.pos > 0 && device_cdf) {
            c = cdf_row(l.row);
        } else if (l.pos > 0) {
            uint32_t* row = cdf_row(lane_index);
            redukt_host::cdf_from_logits_row(logits_row(l.row), vocab, row);
            c = row;
        }
        int32_t st;
        uint32_t tok = 0;
        if (job.mode == Mode::Encode && l.pos > 0 && device_cdf && sym_cdf) {
            tok = job.tokens[l.file][l.pos];
            const uint32_t* b = bounds.data() + size_t(l.row) * 3;
            st = tok < vocab ? l.enc.encode(b[0], b[1], b[2]) : REDUKT_CODEC_INVALID_ARG;  // as encode_symbol
        } else if (job.mode == Mode::Encode) {
            tok = job.tokens[l.file][l.pos];
            st = l.enc.encode_symbol(tok, c, vocab);
        } else if (l.pos > 0 && device_cdf && find_cdf) {
            // Phase B took the target for a total of REDUKT_CDF_TOTAL, the total of every
            // device row; a row that says otherwise is refused like a CDF that does not end
            // at its total.
            const uint32_t* b = bounds.data() + size_t(l.row) * 4;
            st = l.target_status != REDUKT_CODEC_OK ? l.target_status
                 : b[3] != REDUKT_CDF_TOTAL         ? REDUKT_CODEC_INVALID_ARG
                                                    : l.dec.finish(b[0], b[1], b[2], b[3], vocab, vocab, &tok);
            if (st == REDUKT_CODEC_OK) job.tokens_out[l.file][l.pos] = tok;
        } else {
            st = l.dec.decode(c, vocab, vocab, &tok);
            if (st == REDUKT_CODEC_OK) job.tokens_out[l.file][l.pos] = tok;
        }
        if (st != REDUKT_CODEC_OK) {
            l.status = st;
            l.done = true;
            return;
        }
        l.next_token = tok;
        ++l.pos;
        l.done = l.pos >= job.n_tokens[l.file];
    }

    void start_file(const Job& job, Lane& l, int64_t file) {
        l.file = file;
        l.pos = 0;
        l.done = false;
        l.status = REDUKT_CODEC_OK;
        l.since_reset = 0;
        if (job.mode == Mode::Encode)
            l.enc = redukt_rc_encoder();
        else
            l.dec.start(job.streams[file], size_t(job.stream_len[file]));
    }

    void end_file(const Job& job, Lane& l) {
        const int64_t f = l.file;
        int32_t st = l.status;
        if (job.mode == Mode::Encode) {
            if (st == REDUKT_CODEC_OK) {
                l.enc.finish();
                const uint64_t len = l.enc.out.size();
                job.out_len[f] = len;
                if (len <= job.cap[f])
                    std::memcpy(job.out[f], l.enc.out.data(), size_t(len));
                else
                    st = REDUKT_CODEC_BUFFER_TOO_SMALL;
            } else {
                job.out_len[f] = 0;
            }
            l.enc = redukt_rc_encoder();
        }
        if (job.status) job.status[f] = st;
        l.file = -1;
    }

    int32_t run_lockstep(const Job& job, redukt_lockstep_stats& stats);
    int32_t run_compress_pipelined(const Job& job, redukt_lockstep_stats& stats);
    int32_t run_single(const Job& job, redukt_lockstep_stats& stats);
};

namespace {

int32_t overall(const Job& job, const std::vector<int32_t>& st) {
    for (uint32_t f = 0; f < job.n_files; ++f) {
        if (st[f] == REDUKT_CODEC_BUFFER_TOO_SMALL) return REDUKT_LOCKSTEP_BUFFER_TOO_SMALL;
        if (st[f] != REDUKT_CODEC_OK) return REDUKT_LOCKSTEP_CODER;
    }
    return REDUKT_LOCKSTEP_OK;
}

}  // namespace

int32_t redukt_lockstep::run_lockstep(const Job& job, redukt_lockstep_stats& stats) {
    // lockstep.rs:163-265 (run_lockstep).
    std::vector<Lane> lanes(slots);
    std::vector<uint32_t> active, fwd_slots, fwd_tokens, fwd_syms, resets;
    const bool pick = job.mode == Mode::Encode && device_cdf && sym_cdf;
    const bool find = job.mode == Mode::Decode && device_cdf && find_cdf;
    active.reserve(slots);
    uint32_t next_file = 0;
    // The backbone failed: every file still in a lane and every file not yet admitted is
    // marked INCOMPLETE with no output, so a caller reading per-file status never takes a
    // partial file for a finished one.
    auto abort_run = [&]() {
        for (Lane& l : lanes) {
            if (l.file < 0) continue;
            if (job.status) job.status[l.file] = REDUKT_CODEC_INCOMPLETE;
            if (job.mode == Mode::Encode) job.out_len[l.file] = 0;
            l.file = -1;
        }
        for (uint32_t f = next_file; f < job.n_files; ++f) {
            if (job.status) job.status[f] = REDUKT_CODEC_INCOMPLETE;
            if (job.mode == Mode::Encode) job.out_len[f] = 0;
        }
        return REDUKT_LOCKSTEP_FORWARD;
    };
    for (;;) {
        // Admission: every free slot takes the next file, after a reset of its state.
        resets.clear();
        for (uint32_t i = 0; i < slots; ++i) {
            if (lanes[i].file >= 0) continue;
            while (next_file < job.n_files && job.n_tokens[next_file] == 0) {
                if (job.status) job.status[next_file] = REDUKT_CODEC_INVALID_ARG;  // "empty input"
                ++next_file;
            }
            if (next_file >= job.n_files) break;
            start_file(job, lanes[i], next_file++);
            resets.push_back(i);
        }
        if (!resets.empty() && api.batch_reset(resets.data(), uint32_t(resets.size())) != BACKEND_OK)
            return abort_run();
        active.clear();
        for (uint32_t i = 0; i < slots; ++i)
            if (lanes[i].file >= 0) active.push_back(i);
        if (active.empty()) break;

        // Phase A: one unit per active stream on the pool; with the device's three or four
        // values a stream a unit is a few integer operations, less than a hand-over to the
        // pool's threads costs, so the caller codes them all.
        const auto ta = Clock::now();
        redukt_host::parallel_for(active.size(), pick || find ? 1u : threads, [&](size_t k) {
            code_step(job, lanes[active[k]], active[k]);
        });
        stats.tokens += active.size();
        stats.code_secs += since(ta);

        // Finished streams leave their slot before the forward.
        for (uint32_t i : active) {
            if (lanes[i].done) {
                end_file(job, lanes[i]);
                ++stats.files;
            }
        }

        // Phase B: ticks, then one forward_batch for every stream still running.
        const auto tb = Clock::now();
        fwd_slots.clear();
        fwd_tokens.clear();
        fwd_syms.clear();
        resets.clear();
        for (uint32_t i : active) {
            Lane& l = lanes[i];
            if (l.file < 0) continue;
            if (job.reset_every > 0 && l.since_reset >= job.reset_every) {
                resets.push_back(i);
                l.since_reset = 0;
            }
            ++l.since_reset;
            l.row = uint32_t(fwd_slots.size());
            fwd_slots.push_back(i);
            fwd_tokens.push_back(l.next_token);
            if (pick) {
                // the symbol Phase A codes next (an out-of-range one is refused there, per file)
                const uint32_t next = job.tokens[l.file][l.pos];
                fwd_syms.push_back(next < vocab ? next : 0u);
            } else if (find) {
                // the decoder's target for the symbol Phase A decodes next (the state does not
                // change before then); a failure there is that symbol's status
                uint32_t cum = 0;
                l.target_status = l.dec.target(REDUKT_CDF_TOTAL, &cum);
                fwd_syms.push_back(l.target_status == REDUKT_CODEC_OK ? cum : 0u);
            }
        }
        if (!resets.empty() && api.batch_reset(resets.data(), uint32_t(resets.size())) != BACKEND_OK)
            return abort_run();
        if (!fwd_slots.empty()) {
            const uint32_t nf = uint32_t(fwd_slots.size());
            const int32_t rc =
                pick ? api.forward_batch_cdf_sym(nf, fwd_slots.data(), fwd_tokens.data(), fwd_syms.data(), bounds.data(),
                                                 vocab)
                : find ? api.forward_batch_cdf_find(nf, fwd_slots.data(), fwd_tokens.data(), fwd_syms.data(),
                                                    bounds.data(), vocab)
                : device_cdf ? api.forward_batch_cdf(nf, fwd_slots.data(), fwd_tokens.data(), cdf.data(), vocab + 1)
                             : api.forward_batch(nf, fwd_slots.data(), fwd_tokens.data(), logits.data(), vocab);
            if (rc != BACKEND_OK) return abort_run();
        }
        stats.forward_secs += since(tb);
        ++stats.steps;
    }
    return REDUKT_LOCKSTEP_OK;
}

int32_t redukt_lockstep::run_compress_pipelined(const Job& job, redukt_lockstep_stats& stats) {
    // run_lockstep's compression with the same admissions, ticks, forwards and coding per
    // iteration, reordered: a file's tokens are known in advance, so which lanes step
    // next, and on which tokens, follows from the lengths alone.  Iteration i queues its
    // forward before it codes with the results of iteration i - 1's forward.  A lane whose
    // coding fails (an out-of-range token) leaves after that forward was queued with a
    // stand-in token; its slot is reset before it takes another file, and no other
    // stream's results depend on it.
    std::vector<Lane> lanes(slots);
    std::vector<uint32_t> active, fwd_slots, fwd_tokens, fwd_syms, resets;
    active.reserve(slots);
    uint32_t next_file = 0;
    uint64_t pending = 0;   // ticket of the forward whose results the next coding uses
    uint32_t pending_n = 0;
    auto abort_run = [&]() {
        if (pending) (void)api.cdf_sym_wait(pending, bounds.data(), pending_n);
        for (Lane& l : lanes) {
            if (l.file < 0) continue;
            if (job.status) job.status[l.file] = REDUKT_CODEC_INCOMPLETE;
            job.out_len[l.file] = 0;
            l.file = -1;
        }
        for (uint32_t f = next_file; f < job.n_files; ++f) {
            if (job.status) job.status[f] = REDUKT_CODEC_INCOMPLETE;
            job.out_len[f] = 0;
        }
        return REDUKT_LOCKSTEP_FORWARD;
    };
    for (;;) {
        resets.clear();
        for (uint32_t i = 0; i < slots; ++i) {
            if (lanes[i].file >= 0) continue;
            while (next_file < job.n_files && job.n_tokens[next_file] == 0) {
                if (job.status) job.status[next_file] = REDUKT_CODEC_INVALID_ARG;  // "empty input"
                ++next_file;
            }
            if (next_file >= job.n_files) break;
            start_file(job, lanes[i], next_file++);
            resets.push_back(i);
        }
        if (!resets.empty() && api.batch_reset(resets.data(), uint32_t(resets.size())) != BACKEND_OK)
            return abort_run();
        active.clear();
        for (uint32_t i = 0; i < slots; ++i)
            if (lanes[i].file >= 0) active.push_back(i);
        if (active.empty()) break;

        // What Phase A will code, and how far it takes each lane.
        const auto tb = Clock::now();
        fwd_slots.clear();
        fwd_tokens.clear();
        fwd_syms.clear();
        resets.clear();
        for (uint32_t i : active) {
            Lane& l = lanes[i];
            l.code_pos = l.pos;
            l.code_row = l.row;
            l.leaves = l.pos + 1 >= job.n_tokens[l.file];
        }
        // Phase B (ticks, then the forward) for the lanes that go on, queued first.
        for (uint32_t i : active) {
            Lane& l = lanes[i];
            if (l.leaves) continue;
            if (job.reset_every > 0 && l.since_reset >= job.reset_every) {
                resets.push_back(i);
                l.since_reset = 0;
            }
            ++l.since_reset;
            l.row = uint32_t(fwd_slots.size());
            fwd_slots.push_back(i);
            const uint32_t tok = job.tokens[l.file][l.code_pos], next = job.tokens[l.file][l.code_pos + 1];
            fwd_tokens.push_back(tok < vocab ? tok : 0u);   // an out-of-range token fails its file below
            fwd_syms.push_back(next < vocab ? next : 0u);
        }
        // A tick or forward that fails ends the run after this iteration's coding, as in
        // run_lockstep, where they come after it.
        uint64_t ticket = 0;
        const uint32_t nf = uint32_t(fwd_slots.size());
        bool queued = resets.empty() || api.batch_reset(resets.data(), uint32_t(resets.size())) == BACKEND_OK;
        queued = queued && (nf == 0 || api.cdf_sym_submit(nf, fwd_slots.data(), fwd_tokens.data(), fwd_syms.data(),
                                                          vocab, &ticket) == BACKEND_OK);
        if (!queued) ticket = 0;
        // Phase A with the previous forward's results.
        if (pending) {
            const int32_t rc = api.cdf_sym_wait(pending, bounds.data(), pending_n);
            pending = 0;
            if (rc != BACKEND_OK) {
                pending = ticket;
                pending_n = nf;
                return abort_run();
            }
        }
        pending = ticket;
        pending_n = nf;
        stats.forward_secs += since(tb);
        ++stats.steps;
        const auto ta = Clock::now();
        for (uint32_t i : active) {
            Lane& l = lanes[i];
            const uint32_t tok = job.tokens[l.file][l.code_pos];
            int32_t st;
            if (l.code_pos == 0)
                st = l.enc.encode_symbol(tok, uniform.data(), vocab);
            else {
                const uint32_t* b = bounds.data() + size_t(l.code_row) * 3;
                st = tok < vocab ? l.enc.encode(b[0], b[1], b[2]) : REDUKT_CODEC_INVALID_ARG;  // as encode_symbol
            }
            if (st != REDUKT_CODEC_OK) {
                l.status = st;
                l.done = true;
            } else {
                l.next_token = tok;
                l.pos = l.code_pos + 1;
                l.done = l.leaves;
            }
        }
        stats.tokens += active.size();
        stats.code_secs += since(ta);
        for (uint32_t i : active) {
            if (lanes[i].done) {
                end_file(job, lanes[i]);
                ++stats.files;
            }
        }
        if (!queued) return abort_run();
    }
    return REDUKT_LOCKSTEP_OK;
}

int32_t redukt_lockstep::run_single(const Job& job, redukt_lockstep_stats& stats) {
    // The single-file path of the plugin backbone: the v1 global state, one file after
    // the other (codec.rs:1227-1300 with the plugin's forward_into and tick).
    Lane l;
    for (uint32_t f = 0; f < job.n_files; ++f) {
        if (job.n_tokens[f] == 0) {
            if (job.status) job.status[f] = REDUKT_CODEC_INVALID_ARG;
            continue;
        }
        start_file(job, l, f);
        api.reset_state();
        for (;;) {
            const auto ta = Clock::now();
            code_step(job, l, 0);
            stats.code_secs += since(ta);
            ++stats.tokens;
            if (l.done) break;
            const auto tb = Clock::now();
            if (job.reset_every > 0 && l.since_reset >= job.reset_every) {
                api.reset_state();
                l.since_reset = 0;
            }
            ++l.since_reset;
            l.row = 0;
            if (api.forward(l.next_token, logits.data(), vocab) != BACKEND_OK) {
                for (uint32_t g = f; g < job.n_files; ++g) {
                    if (job.status) job.status[g] = REDUKT_CODEC_INCOMPLETE;
                    if (job.mode == Mode::Encode) job.out_len[g] = 0;
                }
                return REDUKT_LOCKSTEP_FORWARD;
            }
            stats.forward_secs += since(tb);
            ++stats.steps;
        }
        end_file(job, l);
        ++stats.files;
    }
    return REDUKT_LOCKSTEP_OK;
}

namespace {

int32_t run(redukt_lockstep* ls, const Job& job, redukt_lockstep_stats* stats_out) {
    redukt_lockstep_stats stats{};
    std::vector<int32_t> st(job.n_files, REDUKT_CODEC_OK);
    Job j = job;
    j.status = st.data();
    const auto t0 = Clock::now();
    int32_t rc = !ls->slots ? ls->run_single(j, stats)
                 : job.mode == Mode::Encode && ls->device_cdf && ls->pipeline ? ls->run_compress_pipelined(j, stats)
                                                                               : ls->run_lockstep(j, stats);
    stats.secs = since(t0);
    if (rc == REDUKT_LOCKSTEP_OK) rc = overall(j, st);
    if (job.status) std::memcpy(job.status, st.data(), st.size() * sizeof(int32_t));
    if (stats_out) *stats_out = stats;
    return rc;
}

}  // namespace

extern "C" int32_t redukt_lockstep_open(const char* plugin_path, const char* weights_path, int32_t device_id,
                                        int32_t profile, uint32_t slots, uint32_t threads, redukt_lockstep** out) {
    if (!out) return REDUKT_LOCKSTEP_INVALID_ARG;
    *out = nullptr;
    if (!plugin_path || !weights_path || slots > BACKEND_MAX_STREAMS) return REDUKT_LOCKSTEP_INVALID_ARG;
    std::unique_ptr<redukt_lockstep> ls(new (std::nothrow) redukt_lockstep());
    if (!ls) return REDUKT_LOCKSTEP_INVALID_ARG;
    if (!ls->api.load(plugin_path)) {
        if (ls->api.handle) dlclose(ls->api.handle);
        return REDUKT_LOCKSTEP_PLUGIN_LOAD;
    }
    auto fail = [&](int32_t code) {
        dlclose(ls->api.handle);
        return code;
    };
    if (slots > 1 && !ls->api.v2) return fail(REDUKT_LOCKSTEP_NEEDS_V2);
    if (slots == 1 && !ls->api.v2) slots = 0;  // one stream on a v1 plugin: the global state
    const auto* path = reinterpret_cast<const uint8_t*>(weights_path);
    int32_t rc;
    if (profile >= 0) {
        if (!ls->api.init_ex) return fail(REDUKT_LOCKSTEP_PLUGIN_LOAD);
        rc = ls->api.init_ex(path, device_id, uint32_t(profile), &ls->info);
    } else {
        rc = ls->api.init(path, device_id, &ls->info);
    }
    if (rc != BACKEND_OK) return fail(REDUKT_LOCKSTEP_PLUGIN_INIT);
    ls->vocab = ls->info.vocab_size;
    if (ls->vocab == 0 || ls->vocab >= REDUKT_CDF_TOTAL) {
        ls->api.free_all();
        return fail(REDUKT_LOCKSTEP_PLUGIN_INIT);
    }
    if (slots > 0 && ls->api.batch_init(slots) != BACKEND_OK) {
        ls->api.free_all();
        return fail(REDUKT_LOCKSTEP_PLUGIN_INIT);
    }
    ls->slots = slots;
    ls->threads = threads;
    const size_t rows = slots ? slots : 1;
    ls->logits.assign(rows * ls->vocab, 0.0f);
    ls->cdf.assign(rows * (size_t(ls->vocab) + 1), 0u);
    ls->uniform.assign(size_t(ls->vocab) + 1, 0u);
    redukt_cdf_uniform(ls->vocab, ls->uniform.data());
    // The device CDF is the faster path wherever the plugin has it (Mamba-130M int8, 16 host
    // threads: forward_batch_cdf 0.93 ms per step at 32 streams against 0.58 ms forward +
    // 0.71 ms host CDF, 1.77 ms at 128 streams against 1.27 + 2.60 ms).
    ls->device_cdf = ls->api.forward_batch_cdf != nullptr && slots >= kDeviceCdfFrom;
    // REDUKT_LOCKSTEP_CDF_SYM=0: compression and decompression take whole device CDF rows.
    const char* e = getenv("REDUKT_LOCKSTEP_CDF_SYM");
    const bool rows_only = e && *e && !strcmp(e, "0");
    ls->sym_cdf = ls->api.forward_batch_cdf_sym != nullptr && !rows_only;
    ls->find_cdf = ls->api.forward_batch_cdf_find != nullptr && !rows_only;
    // REDUKT_LOCKSTEP_PIPELINE=0: compression waits for each step before queueing the next.
    const char* pe = getenv("REDUKT_LOCKSTEP_PIPELINE");
    ls->pipeline = ls->sym_cdf && ls->api.cdf_sym_submit && ls->api.cdf_sym_wait && !(pe && *pe && !strcmp(pe, "0"));
    ls->bounds.assign(rows * 4, 0u);
    *out = ls.release();
    return REDUKT_LOCKSTEP_OK;
}

extern "C" int32_t redukt_lockstep_set_device_cdf(redukt_lockstep* ls, int32_t on) {
    if (!ls) return REDUKT_LOCKSTEP_INVALID_ARG;
    if (on && (!ls->api.forward_batch_cdf || ls->slots == 0)) return REDUKT_LOCKSTEP_INVALID_ARG;
    ls->device_cdf = on != 0;
    return REDUKT_LOCKSTEP_OK;
}

extern "C" int32_t redukt_lockstep_device_cdf(const redukt_lockstep* ls) { return ls && ls->device_cdf ? 1 : 0; }

extern "C" void redukt_lockstep_close(redukt_lockstep* ls) {
    if (!ls) return;
    ls->api.free_all();
    dlclose(ls->api.handle);
    delete ls;
}

extern "C" uint32_t redukt_lockstep_vocab(const redukt_lockstep* ls) { return ls ? ls->vocab : 0; }

extern "C" const char* redukt_lockstep_backend_name(const redukt_lockstep* ls) {
    if (!ls) return "";
    return reinterpret_cast<const char*>(ls->info.name);
}

extern "C" uint64_t redukt_lockstep_stream_bound(uint64_t n_tokens) { return (n_tokens * 25 + 7) / 8 + 5; }

extern "C" int32_t redukt_lockstep_compress(redukt_lockstep* ls, uint32_t n_files, const uint32_t* const* tokens,
                                            const uint64_t* n_tokens, uint64_t reset_every, uint8_t* const* out,
                                            const uint64_t* cap, uint64_t* out_len, int32_t* status,
                                            redukt_lockstep_stats* stats) {
    if (!ls || (n_files && (!tokens || !n_tokens || !out || !cap || !out_len))) return REDUKT_LOCKSTEP_INVALID_ARG;
    for (uint32_t f = 0; f < n_files; ++f)
        if (n_tokens[f] && (!tokens[f] || !out[f])) return REDUKT_LOCKSTEP_INVALID_ARG;
    Job job{Mode::Encode, n_files, n_tokens, reset_every};
    job.tokens = tokens;
    job.out = out;
    job.cap = cap;
    job.out_len = out_len;
    job.status = status;
    return run(ls, job, stats);
}

extern "C" int32_t redukt_lockstep_decompress(redukt_lockstep* ls, uint32_t n_files, const uint8_t* const* streams,
                                              const uint64_t* stream_len, const uint64_t* n_tokens,
                                              uint64_t reset_every, uint32_t* const* tokens_out, int32_t* status,
                                              redukt_lockstep_stats* stats) {
    if (!ls || (n_files && (!streams || !stream_len || !n_tokens || !tokens_out))) return REDUKT_LOCKSTEP_INVALID_ARG;
    for (uint32_t f = 0; f < n_files; ++f)
        if (n_tokens[f] && (!tokens_out[f] || (stream_len[f] && !streams[f]))) return REDUKT_LOCKSTEP_INVALID_ARG;
    Job job{Mode::Decode, n_files, n_tokens, reset_every};
    job.streams = streams;
    job.stream_len = stream_len;
    job.tokens_out = tokens_out;
    job.status = status;
    return run(ls, job, stats);
}
