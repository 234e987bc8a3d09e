/* slm_model.h — the model twin.
 *
 * A C++ restatement of the reference's src/model.rs that drives the C ABI of slm_hip.h
 * exactly as model.rs drives the `Ops` trait: the same calls, in the same order, with the
 * same buffers, including the grow-only output sizing of src/cuda.rs:122-127. It is not
 * part of the drop-in boundary; it stands in for model.rs on top of a Rust `impl Ops for
 * Hip` where no Rust toolchain exists, so tests and benchmarks exercise the backend
 * through the very call sequence the reference makes.
 *
 * Every function returns SLM_OK or a negative SLM_E_* code; slm_model_error gives the
 * message of the last failure on that model or its sessions.
 */
#ifndef SLM_MODEL_H
#define SLM_MODEL_H

#include <stddef.h>
#include <stdint.h>

#include "slm_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct slm_model slm_model;
typedef struct slm_session slm_session;

/* Model::load (model.rs:226-269): config.json and f32 model.safetensors from `dir`. */
int slm_model_load(slm_hip* ctx, const char* dir, slm_model** out);
void slm_model_free(slm_model* m);
/* The last failure on m or its sessions; with m NULL, the last failed slm_model_load. */
const char* slm_model_error(const slm_model* m);
/* Model::params (model.rs:275-302). */
size_t slm_model_params(const slm_model* m);
/* Initial slots of global-layer caches (model.rs:320 uses 8192); for tests of grow. */
int slm_model_set_global_cap(slm_model* m, size_t cap);
/* How a global cache doubles (model.rs:383-398). 0 (the default): model.rs's own sequence —
 * slm_hip_read of each cache inside the advance, the per-head relayout on the host, a fresh
 * upload, the old buffer freed. 1: the relayout as device copies on the stream (the same
 * contents; no host round trip). */
int slm_model_set_device_grow(slm_model* m, int on);

/* Model::session (model.rs:333-381); loops 0 takes the model's default (config.rs:96-105). */
int slm_session_new(slm_model* m, size_t loops, slm_session** out);
void slm_session_free(slm_session* s);
size_t slm_session_pos(const slm_session* s);
size_t slm_session_loops(const slm_session* s);
/* Model::feed (model.rs:656-667). */
int slm_session_feed(slm_session* s, const uint32_t* tokens, size_t n, size_t limit);
/* Model::advance (model.rs:562-640), up to 256 tokens. */
int slm_session_advance(slm_session* s, const uint32_t* tokens, size_t n, int want_logits);
/* Model::step (model.rs:642-645). */
int slm_session_step(slm_session* s, uint32_t token);
/* Model::logits (model.rs:669-671): vocab_size floats. */
int slm_session_logits(slm_session* s, float* out);
/* Model::state_bytes (model.rs:673-690). */
size_t slm_session_state_bytes(const slm_session* s);
/* The buffers passed to flush (model.rs:626-638), logits first: count, lengths (the
 * length the reference's CPU backend would give them), contents. */
size_t slm_session_kept_count(const slm_session* s);
size_t slm_session_kept_len(const slm_session* s, size_t i);
int slm_session_kept_read(slm_session* s, size_t i, float* out, size_t n);
/* sample.rs:48-53's greedy pick on the host: the index b that b = 0, b = i whenever l[i] >
 * l[b] ends on (the first maximum; NaNs never win, a NaN at index 0 keeps 0). A host function:
 * no context or device. */
size_t slm_pick_greedy(const float* logits, size_t n);
/* The decode loop of src/main.rs:207-223: n times, read the logits, pick greedily
 * (slm_pick_greedy) and step; ids[i] receives each pick. */
int slm_session_decode_greedy(slm_session* s, size_t n, uint32_t* ids);
/* The same loop with the pick on the device (replaces the per-token logits read-back and host
 * scan of main.rs:219-222 and sample.rs:48-53 for greedy decoding): each step's logits GEMV is
 * followed by slm_hip_argmax into a device slot that the next step's embedding gather reads,
 * so the steps run back to back with no host round trip; the n ids are read once at the end.
 * The same ids as slm_session_decode_greedy (sample.rs:48-53 semantics). */
int slm_session_decode_greedy_device(slm_session* s, size_t n, uint32_t* ids);

#ifdef __cplusplus
}
#endif

#endif /* SLM_MODEL_H */
