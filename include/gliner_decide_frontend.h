/*
 * gliner_decide_frontend.h -- C-ABI of the decision front end: text + task
 * schema -> one row of classifier input (CPU, libgliner_decide_frontend.so).
 *
 * It stands in for `NativeDecisionTokenizer` (NativeTokenizer.swift:56-227 in
 * shantanugoel/gliner-decide-metal), which formats the classification schema,
 * splits the text into words, cuts out added tokens and runs the rest through
 * the checkpoint's tokenizer.json (a sentencepiece Unigram model behind a
 * Strip / Precompiled / Replace normaliser and a Metaspace pre-tokenizer).
 *
 * Conventions (as gliner_decide.h): every function returns a gd_status
 * (0 = GD_OK) and on failure gd_frontend_last_error() returns a message
 * (thread-local).  Text arguments are UTF-8 byte ranges (not NUL-terminated);
 * invalid UTF-8 is GD_ERR_INVALID_ARGUMENT.  Output arrays are caller-owned
 * host memory; when one is too small the call returns GD_ERR_SHAPE and still
 * reports the size it needs.  A handle may be used from several threads:
 * the calls that use its entry cache (append_tokenized, make_input,
 * clear_cache) take its lock; the others only read it.
 */
#ifndef GLINER_DECIDE_FRONTEND_H_
#define GLINER_DECIDE_FRONTEND_H_

#include <stddef.h>
#include <stdint.h>

#include "gliner_decide.h"

#ifdef __cplusplus
extern "C" {
#endif

#pragma GCC visibility push(default)

/* NativeTokenizerError (NativeTokenizer.swift:5-23) as status codes. */
#define GD_ERR_TOKENIZER_FILES -20    /* .missingTokenizerFiles(directory)          */
#define GD_ERR_TOKENIZER_CONFIG -21   /* .invalidTokenizerConfiguration             */
#define GD_ERR_NO_TASK_LABELS -22     /* .noTaskLabels                              */
#define GD_ERR_INPUT_DOES_NOT_FIT -23 /* .inputDoesNotFit(buckets)                  */

typedef struct gd_frontend gd_frontend;

const char* gd_frontend_last_error(void);

/* NativeDecisionTokenizer(directory:) (NativeTokenizer.swift:63-75, 210-264):
 * reads <directory>/tokenizer.json and requires <directory>/
 * tokenizer_config.json to be a JSON object.  Added tokens ("added_tokens")
 * are the special tokens the front end cuts out; the pad id is that of
 * "[PAD]" (an added token, else the vocabulary's, else 0).  A tokenizer.json
 * component this build does not implement is GD_ERR_UNSUPPORTED. */
int gd_frontend_open(gd_frontend** out, const char* directory);
/* The same from tokenizer.json text already in memory. */
int gd_frontend_create(gd_frontend** out, const char* tokenizer_json, size_t length);
void gd_frontend_destroy(gd_frontend* frontend);
int gd_frontend_pad_id(gd_frontend* frontend, int32_t* pad_id);
/* Empties the handle's entry cache (the ids of recent schema entries and
 * words, at most 65536, emptied when full). */
int gd_frontend_clear_cache(gd_frontend* frontend);

/* The tokenizer pipeline on one text with no added-token cut: the ids of
 * swift-transformers' tokenize + convertTokensToIds (NativeTokenizer.swift:
 * 183-190).  *count = number of ids. */
int gd_frontend_encode(gd_frontend* frontend, const char* text, size_t length, int32_t* ids, int64_t capacity,
                       int64_t* count);

/* appendTokenized (NativeTokenizer.swift:159-181): added tokens cut out
 * first (leftmost occurrence, the longer token on a tie), the text between
 * them through gd_frontend_encode. */
int gd_frontend_append_tokenized(gd_frontend* frontend, const char* text, size_t length, int32_t* ids,
                                 int64_t capacity, int64_t* count);

/* splitWords (NativeTokenizer.swift:193-208): the lower-cased words of a
 * text, each followed by a NUL byte in `buffer`; *bytes = bytes written,
 * *count = words. */
int gd_frontend_split_words(gd_frontend* frontend, const char* text, size_t length, char* buffer, int64_t capacity,
                            int64_t* bytes, int64_t* count);

/* makeInput(text:tasks:buckets:) (NativeTokenizer.swift:76-157) for one
 * example.  tasks_json: a JSON array of DecisionTask objects
 * {"name": s, "labels": [s...], "multiLabel": b?, "prompt": s?,
 *  "labelDescriptions": {label: s}?} (NativeTokenizer.swift:25-44).
 * Outputs: *bucket = L (the smallest bucket >= the encoded length),
 * *length = unpadded length, *heads = Hh = tasks, *options = O = the largest
 * label count; input_ids [L] int32 (right-padded with the pad id),
 * attention_mask [L] fp16 bits (1.0 / 0.0), marker_indices [Hh * O] int32
 * (token index of each label marker, 0 for an empty slot) and marker_mask
 * [Hh * O] fp32 (1 / 0).  No task, or a task without labels, is
 * GD_ERR_NO_TASK_LABELS; no bucket large enough is
 * GD_ERR_INPUT_DOES_NOT_FIT with *bucket = 0 (length, heads and options are
 * still reported). */
int gd_frontend_make_input(gd_frontend* frontend, const char* text, size_t text_length, const char* tasks_json,
                           size_t tasks_length, const int64_t* buckets, int64_t bucket_count, int32_t* input_ids,
                           uint16_t* attention_mask, int64_t capacity, int32_t* marker_indices, float* marker_mask,
                           int64_t marker_capacity, int64_t* bucket, int64_t* length, int64_t* heads,
                           int64_t* options);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* GLINER_DECIDE_FRONTEND_H_ */
