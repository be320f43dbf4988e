/*
 * ns_sampling.h -- C ABI of the MI355X (gfx950) token sampler.
 *
 * Drop-in boundary for NanoServe's sampling hot path.  It replaces the body of
 *   Sampler.sample(logits, sampling_params_list, history_token_ids, generators)
 *   (nanoserve/scheduler/sampler.py:21-89)
 * whose only caller is the engine loop (nanoserve/engine/engine.py:247-249).
 * The Python host mirror (Sampler.sample in the package) packs the per-request
 * SamplingParams (nanoserve/config.py:68-79) and histories
 * (nanoserve/engine/engine.py:242-246) into the device arrays below and calls
 * ns_sample on the current HIP stream.
 *
 * Conventions: plain pointers and sizes only; every pointer in
 * ns_sample_args is a DEVICE pointer; the caller owns all memory and the
 * library allocates nothing and never synchronises.  Calls are asynchronous on
 * `stream`.  Functions return NS_OK (0) or an NS_ERR_* code; ns_last_error()
 * returns the calling thread's last message.
 */
#ifndef NS_SAMPLING_H
#define NS_SAMPLING_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NS_ABI_VERSION 10

#define NS_OK 0
#define NS_ERR_INVALID 1   /* bad argument (message says which) */
#define NS_ERR_ALIGN 2     /* logits rows not 16-byte aligned */
#define NS_ERR_HIP 3       /* a HIP runtime call failed */

#define NS_DTYPE_F32 0
#define NS_DTYPE_BF16 1

#define NS_MODE_AUTO 0        /* per-row once the batch fills the GPU, else segmented (needs a workspace) */
#define NS_MODE_SEGMENTED 1   /* greedy and small-k rows split over several workgroups (needs a workspace) */
#define NS_MODE_PER_ROW 2     /* one workgroup per row for every row */

#define NS_PENALTY_DIVIDE 0      /* penalty_rounding: score / p correctly rounded (torch on the CPU) */
#define NS_PENALTY_RECIPROCAL 1  /* penalty_rounding: score * rep_penalty_recip[r] (torch on a GPU) */

#define NS_KIND_GREEDY 1      /* row_kinds: greedy rows (temperature 0) */
#define NS_KIND_SMALL_K 2     /* row_kinds: sampled rows with 1 <= top_k <= 64 and top_k < vocab */
#define NS_KIND_OTHER 4       /* row_kinds: every other sampled row (top-k off, or top_k > 64) */

#define NS_MAX_VOCAB 262144     /* vocab limit (LDS presence bitmap of vocab/8 bytes) */
#define NS_MAX_HISTORY (1 << 20) /* per-row history limit, in ids (the reference's max_model_len is 8192,
                                    config.py:52); longer rows are reported, not sampled */
#define NS_LDS_HISTORY 8192     /* longest history whose distinct ids the general per-row code keeps in
                                   LDS; a call with a larger max_hist keeps them in its workspace (sized
                                   by ns_sample_workspace_bytes from max_hist) and is refused without one */
#define NS_INFO_WORDS 8         /* int32 words per row in out_info */
#define NS_SEG_MAX_ROWS 16384   /* most rows a segmented call takes (AUTO switches to per-row above) */
#define NS_WIDE_MAX_ROWS 4096   /* most rows a call splits over segment workgroups (NS_KIND_OTHER rows) */
#define NS_NOALLOC_SCRATCH_BYTES (80ull << 20)   /* device scratch of ns_sample_noalloc, per GPU */

/* Per-row diagnostics written to out_info[row * NS_INFO_WORDS + w]:
 *   w=0 path (1 greedy, 2 uniform/NaN guard, 3 top-k set, 4 generic set, 5 large draw,
 *       6 top-k set ordered and drawn by the streaming or segmented kernels, 9 error)
 *   w=1 tokens kept after top-k and top-p
 *   w=2 float32 bits of the top-k threshold in scaled logits (-inf when top-k is off)
 *   w=3 tokens kept after top-k
 *   w=4 top-k candidates examined (-1 when not applicable)
 *   w=5 flags: 1 history id out of range (ignored), 2 history too long, 4 sample row out of range,
 *       8 candidate overflow (generic path taken), 16 histogram refinement limit reached,
 *       32 inverse-CDF locate fell back to the last kept token
 *   w=6 float32 bits of the scaled logit at the top-p cut
 *   w=7 token id at the top-p cut
 */

typedef struct ns_sample_args {
  const void*    logits;        /* [n_rows_total, row_stride] float32 or bfloat16; the model's logits
                                   (engine.py:235-236; bf16 is taken directly, no .float() copy) */
  int32_t        dtype;         /* NS_DTYPE_F32 or NS_DTYPE_BF16 */
  int32_t        n_sample;      /* B, rows to sample (len(sampling_params_list), sampler.py:28) */
  int64_t        n_rows_total;  /* rows of `logits` (bounds for sample_idx) */
  int64_t        vocab;         /* V (sampler.py:28) */
  int64_t        row_stride;    /* elements between consecutive logits rows (>= vocab) */
  const int64_t* sample_idx;    /* [B] rows of `logits` to sample, ascending as built at
                                   scheduler.py:240-246; NULL = rows 0..B-1 (engine.py:235 gather fused) */
  const float*   temperature;   /* [B] SamplingParams.temperature; 0 = greedy (sampler.py:41-50) */
  const int32_t* top_k;         /* [B] SamplingParams.top_k; <= 0 or >= V disables (sampler.py:55) */
  const float*   top_p;         /* [B] SamplingParams.top_p; >= 1 disables (sampler.py:63) */
  const float*   rep_penalty;   /* [B] SamplingParams.repetition_penalty; 1 disables (sampler.py:33) */
  const int32_t* hist_offsets;  /* [B+1] CSR offsets into hist_ids, or NULL for no histories */
  const int32_t* hist_ids;      /* token ids of each row's history (history_token_ids, sampler.py:25) */
  int32_t        max_hist;      /* upper bound on any row's history length (sizes LDS and, above
                                   NS_LDS_HISTORY, the workspace), <= NS_MAX_HISTORY */
  const float*   uniforms;      /* [B] uniforms in [0, 1) replacing torch.multinomial's RNG (sampler.py:87) */
  int64_t*       out_ids;       /* [B] sampled token ids (the LongTensor returned at sampler.py:89) */
  float*         out_probs;     /* [B, vocab] final probabilities (sampler.py:76-80), or NULL; greedy rows
                                   are not written.  Debug/parity output, not part of the timed path. */
  int32_t*       out_info;      /* [B, NS_INFO_WORDS] per-row diagnostics, or NULL */
  void*          workspace;     /* device scratch of ns_sample_workspace_bytes() bytes, 256-byte aligned,
                                   zero-filled before its first use; calls of any shape may share it (the
                                   library leaves its persistent counters at zero after every call), one
                                   call at a time (one stream).  NULL: every row takes the
                                   one-workgroup-per-row kernel.  Read in segmented mode and, outside
                                   NS_MODE_PER_ROW, for the NS_KIND_OTHER rows: those are split over
                                   segment workgroups across the whole GPU (batches up to
                                   NS_WIDE_MAX_ROWS rows). */
  uint64_t       workspace_bytes;
  int32_t        mode;          /* NS_MODE_*: which kernels resolve which rows (results are identical) */
  uint32_t       row_kinds;     /* NS_KIND_* bits of the kinds of rows present, or 0 when unknown: a call
                                   declared without NS_KIND_OTHER rows skips the launches for them */
  void*          hist_state;    /* device-resident histories (ns_hist_state_bytes), or NULL.  With it the
                                   histories are read from the state instead of hist_offsets / hist_ids
                                   (both must be NULL): row r's history is the id list of request slot
                                   hist_slot[r], kept on the device across calls (the lists the engine
                                   rebuilds and copies every step, engine.py:242-246) */
  const int32_t* hist_slot;     /* [B] request slot of each row, -1 for a row without history */
  int32_t        hist_n_slots;  /* slots in hist_state */
  int32_t        hist_capacity; /* token ids per slot */
  int32_t        hist_append;   /* nonzero (needs hist_state): the kernel that writes row r's id also
                                   appends it to slot hist_slot[r], as ns_hist_append would after the
                                   call (scheduler.py:281-284), so the next call sees it without a
                                   further launch.  The rows of such a call name distinct slots; rows
                                   with a negative slot or a failed id (-1) append nothing; a full slot
                                   is left unchanged and counted in *hist_overflow.  0: the state is
                                   only read. */
  int32_t*       hist_overflow; /* device int32 counting the full slots of hist_append, or NULL */
  int32_t        penalty_rounding; /* NS_PENALTY_*: how the penalty's positive branch score / p
                                   (sampler.py:37, p a Python float) rounds.  The reference runs it
                                   with torch on its configured device (config.py:63, "cuda" by
                                   default); there torch multiplies by the float32 reciprocal of the
                                   Python float, while on the CPU it divides.  Negative scores are
                                   multiplied by rep_penalty[r] either way. */
  const float*   rep_penalty_recip; /* [B] with NS_PENALTY_RECIPROCAL: each row's fl32(1 / p), the
                                   reciprocal of the float64 penalty rounded once to float32 (what
                                   torch on a GPU multiplies by); not read with NS_PENALTY_DIVIDE */
} ns_sample_args;

/* Version of this ABI (NS_ABI_VERSION). */
int ns_abi_version(void);

/* Sample one token per row: the whole of sampler.py:28-89 (repetition penalty, temperature,
 * top-k, top-p, softmax with the NaN guard, greedy argmax, inverse-CDF draw).  One
 * workgroup per row (greedy and 1 <= top_k <= 64 rows that fit in registers stream in one
 * pass), optionally preceded by a segmented kernel for greedy and small-k rows of small
 * batches (see NS_MODE_*); every launch is enqueued on `stream`.
 * Replaces Sampler.sample (nanoserve/scheduler/sampler.py:21-89). */
int ns_sample(const ns_sample_args* args, hipStream_t stream);

/* ns_sample without a caller workspace, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  args->workspace must be NULL and workspace_bytes 0: the call
 * uses a fixed device array of NS_NOALLOC_SCRATCH_BYTES (80 MiB) that the library holds on
 * each GPU it runs on until the process ends, and allocates nothing.  Calls whose workspace
 * (ns_sample_workspace_bytes) exceeds it are rejected with NS_ERR_INVALID (the benchmark
 * shapes need at most 28 MiB).  The first call on a device takes the array's address there
 * and clears it with one kernel on `stream` (make that first call outside graph capture).
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU (other streams,
 * other threads) race.  Results are those of ns_sample with a workspace. */
int ns_sample_noalloc(const ns_sample_args* args, hipStream_t stream);

/* Workspace bytes ns_sample needs for n_sample rows of this vocab and logits dtype, with
 * histories of up to max_hist ids (the call's max_hist; 0 without histories). */
int ns_sample_workspace_bytes(int32_t n_sample, int64_t vocab, int32_t dtype, int32_t max_hist, uint64_t* bytes);

/* LDS bytes one workgroup of ns_sample needs for this vocab and history bound. */
int ns_sample_lds_bytes(int64_t vocab, int32_t max_hist, int32_t* lds_bytes);

/* Debug output, outside any sampling call: out[r * ld_out + v] (float32, v < vocab) = the
 * penalized, temperature-scaled logit of sampled row r, i.e. the reference's logits after
 * sampler.py:31-38 and :41-51 (the tensor its top-k and softmax read), computed by one of the
 * routines ns_sample's kernels use:
 *   formula 0  the streaming, top-k, split-row and segment kernels (NS_DEBUG_STREAM)
 *   formula 1  the wide path (NS_DEBUG_WIDE)
 *   formula 2  the per-row general code (NS_DEBUG_GENERAL)
 * args as for ns_sample (uniforms, out_ids, mode, workspace and row_kinds are not read; the
 * pointer checks are the same).  A row whose sample index or history is invalid is written
 * as NaN.  No counterpart in the reference, where the tensor is an intermediate. */
#define NS_DEBUG_STREAM 0
#define NS_DEBUG_WIDE 1
#define NS_DEBUG_GENERAL 2
int ns_debug_scaled(const ns_sample_args* args, int32_t formula, float* out, int64_t ld_out, hipStream_t stream);

/* Device-resident histories: one id list per request slot, capacity ids each, laid out as
 * int32 lengths[n_slots] (padded to 256 bytes) then int32 ids[n_slots][capacity].  The
 * caller owns the buffer (zero-filled: every slot empty).  No counterpart in the reference,
 * which rebuilds every history on the host and copies it each step (engine.py:242-246,
 * sampler.py:34); these keep them on the device, appended in place. */
int ns_hist_state_bytes(int32_t n_slots, int32_t capacity, uint64_t* bytes);

/* Set slot `slot`'s history to ids[0..n) (device pointer): a new request's prompt tokens
 * (engine.py:242-243).  n <= capacity.  Asynchronous on stream. */
int ns_hist_assign(void* state, int32_t n_slots, int32_t capacity, int32_t slot, const int32_t* ids, int32_t n,
                   hipStream_t stream);

/* Append token_ids[r] to slot slots[r] for r < n (device pointers): the sampled tokens join
 * their requests' histories for the next call (scheduler.py:281-284 appending to
 * output_token_ids).  Rows with a negative slot are skipped; a full slot is left unchanged
 * and counted in *overflow (device int32, or NULL).  Asynchronous on stream. */
int ns_hist_append(void* state, int32_t n_slots, int32_t capacity, const int32_t* slots, const int64_t* token_ids,
                   int32_t n, int32_t* overflow, hipStream_t stream);

/* The draw's uniforms for seeded requests (SamplingParams.seed, nanoserve/config.py:79, which
 * the reference declares but never reads; its sampler.py:26 accepts per-row generators and
 * ignores them): uniforms[rows ? rows[j] : j] = Philox4x32-10 (Salmon et al., SC 2011) of the
 * counter (steps[j] low, steps[j] high, 0x4E53534D, 0) under the key (seeds[j] low, seeds[j]
 * high), first output word >> 8, times 2^-24: a float32 in [0, 1).  steps[j] is the number of
 * tokens in the row's history, so a request draws the same uniform for the same history on
 * every call and a new one at every decode step.  seeds, steps: n device values; rows: n device
 * row indices, or NULL.  Asynchronous on stream; the uniforms then go to ns_sample. */
int ns_seeded_uniforms(const uint64_t* seeds, const int64_t* steps, const int32_t* rows, int32_t n, float* uniforms,
                       hipStream_t stream);

/* The logits producer in front of ns_sample (bf16 lm_head GEMM, MFMA, fp32 accumulation):
 *   logits[r][v] = bf16_rne( sum_c hidden[rows ? rows[r] : r][c] * weight[v][c] )
 * for r < m, v < n, c < k.  Replaces the step's gather, GEMM and upcast (engine.py:233-236:
 * hidden.index_select(0, sample_indices), compute_logits(...).float(); llama.py:136-143:
 * F.linear(hidden_states, embed_tokens.weight)): the bf16 logits go to ns_sample as they
 * are, so no float32 copy is written or read.
 * hidden: n_hidden bf16 rows of ld_hidden elements; rows: int64[m] device pointer or NULL
 * (without it the first m rows, m <= n_hidden; a gathered index outside [0, n_hidden) gives
 * that logits row as NaN, which the sampler reports as a NaN row, instead of a read out of
 * bounds, where engine.py:234's index_select would raise); weight:
 * (n, ld_weight) bf16, out_features x in_features (the tied embedding's layout); logits:
 * (m, ld_logits) bf16.  k a positive multiple of 64; hidden and weight 16-byte aligned with
 * ld_hidden, ld_weight multiples of 8 and >= k.  Asynchronous on stream. */
int ns_lm_head_bf16(const void* hidden, int64_t ld_hidden, int64_t n_hidden, const int64_t* rows, const void* weight,
                    int64_t ld_weight, void* logits, int64_t ld_logits, int32_t m, int32_t n, int32_t k,
                    hipStream_t stream);

/* Bytes of the packed lm_head weight for n vocab rows of k: the weight as contiguous
 * 32 KB tiles of 256 rows x 64 (the order the GEMM reads them; rows past n zero).  No
 * counterpart in the reference (its lm_head reads the (n, k) weight as stored). */
int ns_lm_head_packed_bytes(int32_t n, int32_t k, uint64_t* bytes);

/* Pack the (n, ld_weight) bf16 lm_head weight into `packed` (ns_lm_head_packed_bytes bytes,
 * 16-byte aligned), once, at model load: a one-time copy that lets ns_lm_head_bf16_packed
 * stream the weight at close to the HBM rate.  Asynchronous on stream.  No counterpart in
 * the reference. */
int ns_lm_head_pack_bf16(const void* weight, int64_t ld_weight, int32_t n, int32_t k, void* packed,
                         hipStream_t stream);

/* ns_lm_head_bf16 over the packed weight (same result bit for bit: the same products in
 * the same order).  packed_bytes must equal ns_lm_head_packed_bytes(n, k): the buffer was
 * packed for this (n, k).  Replaces the same reference calls (engine.py:233-236,
 * llama.py:136-143). */
int ns_lm_head_bf16_packed(const void* hidden, int64_t ld_hidden, int64_t n_hidden, const int64_t* rows,
                           const void* packed,
                           uint64_t packed_bytes, void* logits, int64_t ld_logits, int32_t m, int32_t n, int32_t k,
                           hipStream_t stream);

/* Last error message of the calling thread ("" if none). */
const char* ns_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NS_SAMPLING_H */
