/* ns_paged_attention.h: C-ABI of the MI355X paged-attention kernels.
 *
 * Replaces the attention step of the reference's decode and chunked-prefill forward:
 *   nanoserve/kernels/paged_attention_triton.py:134-170 (paged_attention_triton: launcher)
 *   nanoserve/kernels/paged_attention_triton.py:19-106  (_paged_attn_kernel: online softmax
 *                                                        over the sequence's KV blocks)
 *   nanoserve/kernels/paged_attention_torch.py:31-100   (paged_attention_torch: the SDPA path)
 * as called from nanoserve/model/attention.py:119-132.
 *
 * Semantics (the reference's): query token i of sequence s (rows query_start_loc[s] ..
 * query_start_loc[s+1]-1, query_lens[s] of them) sits at absolute KV position
 * kv_pos = seq_lens[s] - query_lens[s] + (i - query_start_loc[s]) and attends to KV positions
 * 0 .. min(kv_pos, seq_lens[s]-1) of its sequence; KV position t lives in physical block
 * block_tables[s][t / block_size], slot t % block_size. Query head h reads KV head
 * h / (num_heads_q / num_kv_heads) (GQA). out = softmax(scale * q.K^T) V in float32 arithmetic,
 * rounded to the query's dtype; a query with no visible key gets zeros.
 *
 * Layouts: query/out (total_q, num_heads_q, head_dim), caches (num_blocks, block_size,
 * num_kv_heads, head_dim), each with arbitrary element strides except a unit head_dim stride and
 * 16-byte aligned rows (checked). block_tables int32 (num_seqs, >= max blocks), seq_lens,
 * query_lens int32 (num_seqs), query_start_loc int32 (num_seqs + 1). All pointers are device
 * pointers; nothing is read on the host and no call synchronizes.
 */
#ifndef NS_PAGED_ATTENTION_H
#define NS_PAGED_ATTENTION_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NS_PA_ABI_VERSION 3

#define NS_PA_DTYPE_F32 0
#define NS_PA_DTYPE_BF16 1
#define NS_PA_DTYPE_F16 2

/* query columns of a prefill tile: a tile holds 1 .. NS_PA_TILE_COLUMNS / (num_heads_q /
   num_kv_heads) consecutive query tokens of one sequence */
#define NS_PA_TILE_COLUMNS 128

/* status bits written (OR-ed) by the kernels when args->status is not NULL */
#define NS_PA_STATUS_BAD_BLOCK 1   /* a block table entry outside [0, num_blocks), or a position past
                                      max_blocks_per_seq blocks: that key is skipped */
#define NS_PA_STATUS_SEQ_TOO_LONG 2 /* a sequence needs more KV partitions than max_seq_len sized the
                                       grid for: that query's output is undefined */
#define NS_PA_STATUS_BAD_TILE 4     /* a prefill tile that is not 1 .. tile-width consecutive query tokens
                                       of one sequence, or a listed decode token outside the batch:
                                       skipped, its outputs not written */

typedef struct ns_paged_attn_args {
  const void*    query;            /* (total_q, num_heads_q, head_dim), dtype */
  const void*    k_cache;          /* (num_blocks, block_size, num_kv_heads, head_dim), dtype */
  const void*    v_cache;          /* same shape and dtype as k_cache */
  void*          out;              /* (total_q, num_heads_q, head_dim), dtype */
  const int32_t* block_tables;     /* (num_seqs, stride_bt_seq) */
  const int32_t* seq_lens;         /* (num_seqs) */
  const int32_t* query_start_loc;  /* (num_seqs + 1) */
  const int32_t* query_lens;       /* (num_seqs) */
  int32_t*       status;           /* optional, one word: NS_PA_STATUS_* bits */
  void*          workspace;        /* ns_paged_attention_workspace_bytes() bytes, or NULL if 0 */
  uint64_t       workspace_bytes;
  int32_t*       counters;         /* when the workspace is needed: total_q * num_kv_heads arrival
                                      counters, zero-filled before first use and left zeroed by
                                      every call (whatever its shape), so one buffer serves all
                                      calls of one stream */
  int64_t        stride_q_token, stride_q_head;
  int64_t        stride_k_block, stride_k_token, stride_k_head;
  int64_t        stride_v_block, stride_v_token, stride_v_head;
  int64_t        stride_o_token, stride_o_head;
  int64_t        stride_bt_seq;
  int32_t        total_q;
  int32_t        num_seqs;
  int32_t        num_heads_q;
  int32_t        num_kv_heads;
  int32_t        head_dim;         /* 64 or 128 */
  int32_t        block_size;
  int32_t        num_blocks;
  int32_t        max_blocks_per_seq; /* valid columns of block_tables (entries past it are not read) */
  int32_t        max_seq_len;      /* >= every seq_lens[s]; sizes the grid and the workspace */
  int32_t        dtype;            /* NS_PA_DTYPE_* */
  float          scale;
  /* Query tiles for sequences with several query tokens (chunked prefill), bfloat16 and float16
   * only: prefill_tiles holds n_prefill_tiles int32 triples (sequence, first query token, token
   * count), each 1 .. NS_PA_TILE_COLUMNS / (num_heads_q / num_kv_heads) consecutive tokens of one sequence; a tile
   * reads each key and value row once for all its tokens and heads (MFMA).  With tiles,
   * decode_tokens lists the n_decode_tokens other query tokens (flat indices), which the per-token
   * kernel takes; every query token belongs to exactly one tile or the list (an unlisted token's
   * output is not written).  prefill_tiles NULL: the per-token kernel takes decode_tokens when it is
   * set, else every token.  Device pointers. */
  const int32_t* decode_tokens;
  int32_t        n_decode_tokens;
  const int32_t* prefill_tiles;
  int32_t        n_prefill_tiles;
} ns_paged_attn_args;

/* Version of this ABI (NS_PA_ABI_VERSION). */
int ns_pa_abi_version(void);

/* Message of the last failed call on this thread. */
const char* ns_pa_last_error(void);

/* Workspace bytes a call with these sizes needs (0 when every query fits one KV partition): the
 * partials of split rows (no initial contents needed). A call that needs a workspace also needs the
 * counters buffer. Returns 0 on success, nonzero on invalid sizes. */
int ns_paged_attention_workspace_bytes(int32_t total_q, int32_t num_heads_q, int32_t num_kv_heads,
                                       int32_t head_dim, int32_t max_seq_len, uint64_t* bytes);

/* Workspace bytes and counter words a call with these arguments needs (prefill tiles included):
 * the counters buffer holds total_q * num_kv_heads words for the per-token kernel, then
 * n_prefill_tiles * num_kv_heads for the tiles; zero-filled once, left zeroed by every call. */
int ns_paged_attention_call_workspace(const ns_paged_attn_args* args, uint64_t* bytes, uint64_t* counters);

/* Paged attention (paged_attention_triton.py:134-170, paged_attention_torch.py:31-100): one
 * launch; one workgroup per (query token, KV head, KV partition) computes all query heads of that
 * KV head, so each key and value row is read once per query token; when a query spans several
 * partitions the last of them to finish merges them. Returns 0 on success, nonzero on invalid
 * arguments. */
int ns_paged_attention(const ns_paged_attn_args* args, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NS_PAGED_ATTENTION_H */
