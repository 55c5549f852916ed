/*
 * oxbitnet.h — the 0xBitNet C ABI, served by liboxbitnet (MI355X / HIP).
 *
 * Drop-in for packages/rust/crates/oxbitnet-ffi/oxbitnet.h of m96-chan/0xBitNet:
 * the same symbols, enum values, struct layouts (LP64) and callback types,
 * so a caller built against the reference header links against this library
 * unchanged.  Each declaration cites the reference line it matches.
 *
 * Semantics kept from the reference implementation (oxbitnet-ffi/src/lib.rs):
 *  - every call clears the thread's last error first; failures return NULL or
 *    -1 and leave a message readable through oxbitnet_error_message() until
 *    the next call on the same thread;
 *  - generate/chat block the calling thread and call the token callback on
 *    it; a non-zero return stops generation; tokens are NUL-terminated and
 *    valid only during the callback; they return 0 even when generation ends
 *    early;
 *  - options == NULL means the defaults, with repeat_penalty 1.1;
 *  - a handle must not be used by two threads at once.
 * Differences: sources are local GGUF paths (there is no HTTP download or
 * cache in this build: a URL fails with an error), and the tokenizer is the
 * byte-level greedy pass-through described in the build's design notes.
 */
#ifndef OXBITNET_H
#define OXBITNET_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ffi/oxbitnet.h:14-18 */
typedef enum OxBitNetLoadPhase {
  Download = 0,
  Parse = 1,
  Upload = 2,
} OxBitNetLoadPhase;

/* ffi/oxbitnet.h:23-29 */
typedef enum OxBitNetLogLevel {
  Trace = 0,
  Debug = 1,
  Info = 2,
  Warn = 3,
  Error = 4,
} OxBitNetLogLevel;

/* ffi/oxbitnet.h:34 — opaque model handle */
typedef struct OxBitNet OxBitNet;

/* ffi/oxbitnet.h:39-42 */
typedef void (*OxBitNetLogFn)(enum OxBitNetLogLevel level, const char *message, uintptr_t len,
                              void *userdata);

/* ffi/oxbitnet.h:47-68 (40 bytes on LP64) */
typedef struct OxBitNetGenerateOptions {
  uintptr_t max_tokens;  /* tokens to generate at most */
  float temperature;     /* 1.0 = unscaled logits */
  uintptr_t top_k;       /* 1 = greedy */
  float repeat_penalty;  /* 1.0 = off */
  uintptr_t repeat_last_n;
} OxBitNetGenerateOptions;

/* ffi/oxbitnet.h:73-78 */
typedef struct OxBitNetLoadProgress {
  enum OxBitNetLoadPhase phase;
  uint64_t loaded;
  uint64_t total;
  double fraction;
} OxBitNetLoadProgress;

/* ffi/oxbitnet.h:83 */
typedef void (*OxBitNetProgressFn)(const struct OxBitNetLoadProgress *progress, void *userdata);

/* ffi/oxbitnet.h:88-101 */
typedef struct OxBitNetLoadOptions {
  OxBitNetProgressFn on_progress; /* nullable */
  void *progress_userdata;        /* nullable */
  const char *cache_dir;          /* nullable; unused (no downloads) */
} OxBitNetLoadOptions;

/* ffi/oxbitnet.h:106 — return 0 to continue, non-zero to stop */
typedef int32_t (*OxBitNetTokenFn)(const char *token, uintptr_t len, void *userdata);

/* ffi/oxbitnet.h:111-120 */
typedef struct OxBitNetChatMessage {
  const char *role;
  const char *content;
} OxBitNetChatMessage;

/* ffi/oxbitnet.h:135 — process-wide; the first call wins, later calls are
 * no-ops.  min_level: 0 Trace .. 4 Error. */
void oxbitnet_set_logger(OxBitNetLogFn callback, void *userdata, uint8_t min_level);

/* ffi/oxbitnet.h:140 — {256, 1.0, 50, 1.1, 64} */
struct OxBitNetGenerateOptions oxbitnet_default_generate_options(void);

/* ffi/oxbitnet.h:145 — {NULL, NULL, NULL} */
struct OxBitNetLoadOptions oxbitnet_default_load_options(void);

/* ffi/oxbitnet.h:161 — NULL on error */
struct OxBitNet *oxbitnet_load(const char *source, const struct OxBitNetLoadOptions *options);

/* ffi/oxbitnet.h:173 — NULL is a no-op */
void oxbitnet_free(struct OxBitNet *model);

/* ffi/oxbitnet.h:190-194 — 0 on success, -1 on error */
int32_t oxbitnet_generate(struct OxBitNet *model, const char *prompt,
                          const struct OxBitNetGenerateOptions *options, OxBitNetTokenFn callback,
                          void *userdata);

/* ffi/oxbitnet.h:211-216 — 0 on success, -1 on error */
int32_t oxbitnet_chat(struct OxBitNet *model, const struct OxBitNetChatMessage *messages,
                      uintptr_t num_messages, const struct OxBitNetGenerateOptions *options,
                      OxBitNetTokenFn callback, void *userdata);

/* ffi/oxbitnet.h:224 — NULL if the last call on this thread succeeded */
const char *oxbitnet_error_message(void);

#ifdef __cplusplus
}
#endif
#endif /* OXBITNET_H */
