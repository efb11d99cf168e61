/* exactsample_amd: C ABI of the MI355X (gfx950) sampling and draft-verification path.
 *
 * Drop-in boundary for the reference's C++ API (include/exactsample/api.h:7-44)
 * and the op binding that fills it (csrc/bindings.cpp:45-136). Plain C types,
 * plain pointers and sizes; no PyTorch types. A thin PyTorch op
 * (exactsample/csrc/binding.cpp) and a ctypes caller both sit on top.
 *
 * Semantics are the reference contract (docs/contract.md): per-request statuses,
 * -1 tokens for failed requests, Philox keyed by (seed, stream, position,
 * substream, token / 4) (docs/rng.md), ties split by token ID.
 */
#ifndef EXACTSAMPLE_AMD_H
#define EXACTSAMPLE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Per-request status codes; replaces exactsample::Status (api.h:8). */
enum es_status { ES_OK = 0, ES_NO_VALID_TOKEN = 1, ES_INVALID_INPUT = 2, ES_DRAFT_ZERO_PROB = 3 };
/* path_used values; replaces exactsample::Path (api.h:9). */
enum es_path { ES_PATH_REFERENCE = 0, ES_PATH_FUSED = 1 };
/* Logit element types; replaces exactsample::DType (api.h:10). */
enum es_dtype { ES_F32 = 0, ES_F64 = 1, ES_F16 = 2, ES_BF16 = 3 };
/* Host-side error codes of es_launch (structural problems; numerical ones are statuses). */
enum es_error {
  ES_SUCCESS = 0,
  ES_ERR_NULL_ARGUMENT = 1,     /* a required pointer is null */
  ES_ERR_BAD_DIMENSION = 2,     /* rows/requests/vocab/max_draft out of the supported range */
  ES_ERR_BAD_OPTION = 3,        /* mode, dispatch or list_max out of range */
  ES_ERR_WORKSPACE_SIZE = 4,    /* workspace smaller than es_workspace_size() */
  ES_ERR_WORKSPACE_ALIGN = 5,   /* workspace not 8-byte aligned */
  ES_ERR_BAD_DTYPE = 6,         /* unknown es_dtype, or draft dtype differs from target */
  ES_ERR_LAUNCH = 7,            /* the HIP runtime refused a kernel launch */
  ES_ERR_STATIC_CAPACITY = 8    /* es_launch_static: the call needs more than ES_STATIC_WORKSPACE_BYTES */
};

/* A [rows, vocab] logits matrix with element strides; replaces exactsample::Matrix (api.h:11-15). */
typedef struct es_matrix {
  const void* data;
  int64_t s0, s1;
  int32_t dtype; /* enum es_dtype */
  int32_t pad;
} es_matrix;

/* A strided vector; replaces exactsample::Vector<T> (api.h:16-19). */
typedef struct es_vec_i64 { const int64_t* data; int64_t stride; } es_vec_i64;
typedef struct es_vec_f64 { const double* data; int64_t stride; } es_vec_f64;

/* Everything one call needs; replaces exactsample::Arguments (api.h:21-36).
 * All pointers are device pointers. Strides are in elements. */
typedef struct es_arguments {
  es_matrix target;        /* [rows, vocab] */
  es_matrix draft;         /* full-q draft logits, same shape and dtype, or data == NULL */
  es_vec_i64 cu_rows;      /* [requests + 1] */
  es_vec_i64 top_k;        /* [requests], 0 disables */
  es_vec_i64 draft_kind;   /* [requests], 0 one-hot, 1 full */
  es_vec_i64 seed;         /* [requests], signed storage of the uint64 key */
  es_vec_i64 stream;       /* [requests], in [0, 2^32) */
  es_vec_i64 position;     /* [rows], in [0, 2^32) */
  es_vec_f64 temperature;  /* [requests] */
  es_vec_f64 top_p;        /* [requests] */
  es_vec_f64 min_p;        /* [requests] */
  const int64_t* draft_ids; int64_t draft_s0, draft_s1;  /* [requests, >= max_draft] */
  const int32_t* mask; int64_t mask_s0, mask_s1;         /* [rows, ceil(vocab/32)] or NULL */
  int64_t* tokens; int64_t token_s0, token_s1;           /* [>= requests, >= max_draft + 1] */
  int32_t* accepted; int64_t accepted_s;                 /* [>= requests] */
  int32_t* status; int64_t status_s;                     /* [>= requests] */
  int32_t* path; int64_t path_s;                         /* [>= requests] */
  int64_t rows, requests, vocab, max_draft;
  int32_t mode;            /* 0 ratio, 1 coupled */
  int32_t dispatch;        /* 0 auto, 1 reference, 2 fused */
  int32_t list_max;        /* largest kept set finished as an FP64 list, 0..256 */
  int32_t pad;
  uint8_t* workspace;      /* es_workspace_size() bytes, zeroed once when allocated */
  uint64_t workspace_bytes;
} es_arguments;

/* Bytes of workspace for `rows` rows; `reference` != 0 adds the dispatch="reference"
 * scratch. Same formula as exactsample::workspace_size (api.h:37-43):
 * 8 + rows * (32 + max(12288, reference ? 20 * vocab : 0)). Returns 0 on overflow. */
size_t es_workspace_size(int64_t rows, int64_t vocab, int32_t reference);

/* Enqueues one call on `stream` (a hipStream_t; NULL is the null stream). Never
 * allocates, never synchronizes. Replaces exactsample::launch (api.h:44,
 * csrc/verify/verify.cu:220-228). Returns an es_error code. */
int32_t es_launch(const es_arguments* args, void* stream);

/* Bytes of the library's own per-GPU workspace used by es_launch_static: room
 * for 8 + rows * 12320 bytes, i.e. up to 1,361 rows of any vocabulary. */
#define ES_STATIC_WORKSPACE_BYTES (16u << 20)

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): es_launch with the workspace replaced by a file-scope
 * device array of ES_STATIC_WORKSPACE_BYTES in this library, one copy per GPU
 * held until the process ends (its address is looked up on the device's first
 * call). args->workspace and args->workspace_bytes are ignored; the caller
 * still passes inputs and outputs. Calls needing more than the array (rows
 * above 1,361) return ES_ERR_STATIC_CAPACITY before any HIP call. No call
 * allocates or frees memory. No byte of the array needs a particular value
 * when a call starts. Every call on one GPU shares that GPU's array: calls
 * that overlap on one GPU (on different streams, or from several host
 * threads) race and must not be issued. The FP64 recomputation count of the
 * last call is not exposed. */
int32_t es_launch_static(const es_arguments* args, void* stream);

/* A static description of an es_error code. */
const char* es_error_string(int32_t code);

/* The last HIP runtime error string seen by es_launch on this thread ("" if none). */
const char* es_last_hip_error(void);

/* Timing hook with no counterpart in the reference, for benchmarks and profilers
 * that want the two kernels of a call timed apart. When `event` (a hipEvent_t) is
 * non-null, every later es_launch on this thread records it on the call's stream
 * between the slice-stream kernel and the per-row finishing kernel; NULL turns it
 * off. Recording adds a stream marker, so leave it off outside measurement. */
void es_set_split_event(void* event);

/* Device self-test with no counterpart in the reference's API; it makes, on this
 * GPU and with this library's build, the checks of the reference's
 * tests/exhaustive/gumbel_bound.cu:33-78 for the FP32 Gumbel noise the certified
 * draws use: over words [first_word, first_word + count) of the 2^32 Philox
 * words, |gumbel32 - G| <= 2^-19 (1 + |G|), the cheap screen >= G, and
 * G < 22.875, where G = -log(-log u) in FP64. `report` is 8 device uint64 words
 * (8-byte aligned), overwritten: words checked, error-bound violations,
 * screen violations, range violations, largest error / bound (FP64 bits),
 * then the smallest screen margin, largest G and smallest G as order keys
 * (key k: FP64 bits k & ~2^63 if k >= 2^63, else ~k). Enqueued on `stream`. */
int32_t es_check_gumbel(uint64_t first_word, uint64_t count, uint64_t* report, void* stream);

/* Device self-test with no counterpart in the reference's API, of the bound
 * the certified FP32 sums and min-p decisions use (the reference states it as
 * X_ERR, csrc/verify/fused.cuh:62-67, for its CUDA expf): over indices
 * [first_index, first_index + count) of [0, 2^32), index i <= 0x42200000 checks
 * the FP32 x with bits 0x80000000 | i (every FP32 x in [-40, 0] over the whole
 * range): |weight32(x) / exp(x) - 1| <= 2.9e-7; every index also checks a
 * pseudo-random (v, M, T): |x32 - x| <= 1.8e-7 |x| + 2^-126 for x32 as the
 * kernels form it and x = (v - M) / T in FP64, and, for x in [-40, 0],
 * |weight32(x32) / exp(x) - 1| <= 4.8e-7 (1 + |x|). `report` is 8 device
 * uint64 words, overwritten: indices checked, weight violations, formation
 * violations, combined violations, then as FP64 bits the largest weight error,
 * the largest |x32 - x| / |x| and the largest combined error / bound, then
 * the count of FP32 x checked. Enqueued on `stream`. */
int32_t es_check_weights(uint64_t first_index, uint64_t count, uint64_t* report, void* stream);

/* Offset of the FP64 recomputation counter in the workspace (a uint32 written by
 * each call; read it after the call completes). Replaces workspace word 1 read at
 * python/exactsample/cuda.py:109-114. */
size_t es_fallback_counter_offset(void);

#ifdef __cplusplus
}
#endif

#endif /* EXACTSAMPLE_AMD_H */
