// Paged attention for gfx950 (decode and chunked prefill).
//
// Follows nanoserve/kernels/paged_attention_triton.py:19-106 (per query token: online softmax over
// the sequence's KV blocks, GQA by h / NUM_KV_GROUPS, causal cut at the query's own KV position,
// zero output when no key is visible) and the launcher's index set-up (:109-131: sequence of each
// query token, its absolute KV position), re-designed for MI355X:
//
//  * One 256-thread workgroup per (query token, KV head, KV partition) computes every query head of
//    that KV head (G = num_heads_q / num_kv_heads of them), so each key and value row is read from
//    HBM once per query token instead of once per query head as the reference's per-(token, head)
//    programs do. Decode attention moves ~4 flops per byte: HBM bound, VALU arithmetic.
//  * Lane layout per wave step: 16 KV positions, 8 lanes per position, each lane holding a
//    head_dim/8 slice (32 contiguous bytes of a bf16 row at head_dim 128: two 16-byte loads). The
//    slice's partial dot products are summed across the 8 lanes with ds_swizzle (no LDS traffic).
//  * Exact two-pass softmax inside a partition: scores (already in log2 units) go to LDS, one max
//    and one exp2 pass over LDS, then the value pass. Partitions of a long sequence (split-KV,
//    sized on the host so that the grid holds >= 1024 workgroups) are merged by the last of the
//    row's workgroups to arrive (max-rescaled sums); a query that fits one partition is written
//    directly. One launch per call.
//  * The sequence of a query token and its KV position are computed in the kernel (binary search
//    over query_start_loc), so a call needs no host copy of the batch layout.

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "ns_paged_attention.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kSub = 2;                 // KV positions per lane per batch
constexpr int kMaxPart = 1024;          // largest KV partition (LDS score buffer)
constexpr int kMinPart = 64;
constexpr int kTargetGroups = 1024;     // workgroups a launch aims for before splitting stops
constexpr float kLog2e = 1.4426950408889634f;

thread_local char g_err[512];

int fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return 1;
}

struct PaParams {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const int32_t* bt;
  const int32_t* seq_lens;
  const int32_t* qsl;
  const int32_t* qlens;
  int32_t* status;
  float* ws_acc;    // (total_q, Hq, max_parts, D) unnormalised partition outputs
  float* ws_ml;     // (total_q, Hq, max_parts, 2) partition max (log2 units) and sum
  int32_t* counters;  // (total_q, Hkv) arrivals of split rows' partitions; zero between calls
                      // (a buffer of its own: any call shape leaves every counter at zero)
  int64_t sq_tok, sq_head, sk_blk, sk_tok, sk_head, sv_blk, sv_tok, sv_head, so_tok, so_head, sbt;
  int32_t num_seqs, hq, hkv, block_size, num_blocks, max_blocks_per_seq, part_tokens, max_parts;
  int32_t total_q;
  const int32_t* tokens;  // the query tokens the decode kernel takes (blockIdx.x indexes it), or NULL: all
  int32_t bs_shift;  // log2(block_size) when it is a power of two, else -1
  float scale_log2;  // scale * log2(e): scores in log2 units, exp2 for the softmax
};

// ---- element loads / stores -------------------------------------------------------------------

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct Bf16 {};
struct F16 {};

template <typename T> struct Elem;
template <> struct Elem<float> { static constexpr int bytes = 4; };
template <> struct Elem<Bf16> { static constexpr int bytes = 2; };
template <> struct Elem<F16> { static constexpr int bytes = 2; };

// N consecutive elements (N * bytes a multiple of 16, 16-byte aligned) as raw 16-byte words ...
template <typename T, int N>
struct Raw {
  static constexpr int kVec = N * Elem<T>::bytes / 16;
  u32x4 w[kVec];
};

template <typename T, int N>
__device__ __forceinline__ void load_raw(const void* base, int64_t elem_off, Raw<T, N>& r) {
  const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + elem_off * Elem<T>::bytes);
#pragma unroll
  for (int i = 0; i < Raw<T, N>::kVec; ++i) r.w[i] = p[i];
}

// ... converted to float
template <typename T, int N>
__device__ __forceinline__ void to_float(const Raw<T, N>& r, float (&x)[N]) {
  const uint32_t* u = reinterpret_cast<const uint32_t*>(r.w);
  if constexpr (Elem<T>::bytes == 4) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = __uint_as_float(u[i]);
  } else if constexpr (__is_same(T, Bf16)) {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      x[2 * i] = __uint_as_float(u[i] << 16);
      x[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(u[i] & 0xFFFFu));
      const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(u[i] >> 16));
      x[2 * i] = (float)lo;
      x[2 * i + 1] = (float)hi;
    }
  }
}

template <typename T>
__device__ __forceinline__ void store_one(void* base, int64_t elem_off, float x) {
  if constexpr (Elem<T>::bytes == 4) {
    reinterpret_cast<float*>(base)[elem_off] = x;
  } else if constexpr (__is_same(T, Bf16)) {
    // round to nearest even; NaN stays a quiet NaN
    uint32_t u = __float_as_uint(x);
    uint16_t h;
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) {
      h = (uint16_t)((u >> 16) | 0x40u);
    } else {
      u += 0x7FFFu + ((u >> 16) & 1u);
      h = (uint16_t)(u >> 16);
    }
    reinterpret_cast<uint16_t*>(base)[elem_off] = h;
  } else {
    reinterpret_cast<_Float16*>(base)[elem_off] = (_Float16)x;
  }
}

// ---- lane exchanges ---------------------------------------------------------------------------

// Sum over the 8 lanes of an aligned lane octet: ds_swizzle in bitmask mode (xor 1, 2, 4).
__device__ __forceinline__ float octet_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x041F));
  x += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x081F));
  x += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x101F));
  return x;
}

// Sum over the 16 lanes of an aligned group (the octet sum, then xor 8).
__device__ __forceinline__ float hex_sum(float x) {
  x = octet_sum(x);
  x += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x201F));
  return x;
}

// Sum over the lanes that share lane % L (xor L, 2L, ... 32).
template <int L>
__device__ __forceinline__ float slot_sum(float x) {
#pragma unroll
  for (int s = L; s < 64; s <<= 1) x += __shfl_xor(x, s);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) x = fmaxf(x, __shfl_xor(x, s));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) x += __shfl_xor(x, s);
  return x;
}

// Stores and loads of the partition partials at agent scope: the workgroups of one row run on
// different XCDs, whose L2s are not coherent with each other for plain accesses.
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- batch layout -----------------------------------------------------------------------------

struct QueryPlace {
  int seq;
  int kv_len;  // visible KV positions: min(kv_pos + 1, seq_len), at least 0
};

// Sequence of query token qi: the largest s with query_start_loc[s] <= qi (empty sequences share
// their start with the next one, so the largest index is the one that owns qi), as the reference's
// repeat_interleave over query_lens (paged_attention_triton.py:109-112); its KV position
// seq_len - q_len + (qi - start) (:115-131), the causal and in-sequence cuts (:64-66).
__device__ __forceinline__ QueryPlace place_query(const PaParams& p, int qi) {
  int lo = 0, hi = p.num_seqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (p.qsl[mid] <= qi) lo = mid; else hi = mid - 1;
  }
  const int seq_len = p.seq_lens[lo];
  const int kv_pos = seq_len - p.qlens[lo] + (qi - p.qsl[lo]);
  int kv_len = kv_pos + 1 < seq_len ? kv_pos + 1 : seq_len;
  if (kv_len < 0) kv_len = 0;
  return {lo, kv_len};
}

// ---- partition kernel ---------------------------------------------------------------------------

template <typename T, int D, int G>
__global__ __launch_bounds__(kThreads) void pa_partition_kernel(PaParams p) {
  // L lanes per KV position, DS dims each: 8 lanes, or 16 for eight heads of 128 dims (the query
  // slices and accumulators of eight heads would not fit the registers at 16 dims a lane)
  constexpr int L = (G == 8 && D == 128) ? 16 : 8;
  constexpr int DS = D / L;           // dims per lane
  constexpr int NSLOT = 64 / L;       // positions a wave covers per row of a batch
  constexpr int kBatch = NSLOT * kSub;  // KV positions per wave batch
  static_assert(G <= L, "the lane with dl == g stores head g's score");
  __shared__ float s_score[G * kMaxPart];
  __shared__ float s_red[kWaves * G * D];
  __shared__ float s_m[G], s_l[G];
  __shared__ int s_blk[kMaxPart + 2];  // physical block of each block-table entry the partition spans

  const int qi = p.tokens != nullptr ? p.tokens[blockIdx.x] : (int)blockIdx.x;
  const int kvh = blockIdx.y, part = blockIdx.z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (qi < 0 || qi >= p.total_q) {   // a listed token outside the batch: flagged, nothing touched
    if (threadIdx.x == 0 && part == 0 && kvh == 0 && p.status) atomicOr(p.status, NS_PA_STATUS_BAD_TILE);
    return;
  }
  const int slot = lane / L;  // position within a row of the batch
  const int dl = lane % L;     // dim slice
  const QueryPlace qp = place_query(p, qi);
  const int n_parts = (qp.kv_len + p.part_tokens - 1) / p.part_tokens;

  if (part == 0 && n_parts > p.max_parts && threadIdx.x == 0 && p.status)
    atomicOr(p.status, NS_PA_STATUS_SEQ_TOO_LONG);
  if (part >= n_parts) {
    if (part == 0) {  // no visible key: zeros (the reference's l == 0 guard, :103-104)
      for (int i = threadIdx.x; i < G * D; i += kThreads)
        store_one<T>(p.out, (int64_t)qi * p.so_tok + (int64_t)(kvh * G + i / D) * p.so_head + i % D, 0.f);
    }
    return;
  }
  const int t0 = part * p.part_tokens;
  const int t1 = min(qp.kv_len, t0 + p.part_tokens);
  const int n = t1 - t0;
  const int32_t* bt_row = p.bt + (int64_t)qp.seq * p.sbt;

  // the partition's slice of the block table, validated once, into LDS
  const int bi0 = t0 / p.block_size;
  const int nbi = (t1 - 1) / p.block_size - bi0 + 1;
  for (int i = threadIdx.x; i < nbi; i += kThreads) {
    const int bi = bi0 + i;
    int blk = bi < p.max_blocks_per_seq ? bt_row[bi] : -1;
    if (blk < 0 || blk >= p.num_blocks) {
      blk = -1;
      if (p.status) atomicOr(p.status, NS_PA_STATUS_BAD_BLOCK);
    }
    s_blk[i] = blk;
  }

  // query slices, pre-scaled into log2 units
  float qv[G][DS];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    Raw<T, DS> r;
    load_raw<T, DS>(p.q, (int64_t)qi * p.sq_tok + (int64_t)(kvh * G + g) * p.sq_head + dl * DS, r);
    to_float<T, DS>(r, qv[g]);
#pragma unroll
    for (int i = 0; i < DS; ++i) qv[g][i] *= p.scale_log2;
  }
  __syncthreads();

  // Position j of the partition for sub-row r of the batch starting at base; its physical block
  // from LDS (-1: past the partition or an invalid entry).
  auto block_of = [&](int j, int& off) -> int {
    if (j >= n) return -1;
    const int t = t0 + j;
    int bi;
    if (p.bs_shift >= 0) {  // the usual case (16): a shift and a mask instead of an integer division
      bi = t >> p.bs_shift;
      off = t & (p.block_size - 1);
    } else {
      bi = t / p.block_size;
      off = t - bi * p.block_size;
    }
    return s_blk[bi - bi0];
  };

  // pass 1: scores -> LDS. A wave takes batches of kBatch positions (wave w: batches w, w + 4, ...);
  // each lane requests its kSub rows of the batch before any arithmetic.
  for (int base = wave * kBatch; base < n; base += kWaves * kBatch) {
    Raw<T, DS> raw[kSub];
    int blk[kSub];
#pragma unroll
    for (int r = 0; r < kSub; ++r) {
      int off = 0;
      blk[r] = block_of(base + r * NSLOT + slot, off);
      if (blk[r] >= 0)
        load_raw<T, DS>(p.k, (int64_t)blk[r] * p.sk_blk + (int64_t)off * p.sk_tok + (int64_t)kvh * p.sk_head + dl * DS,
                        raw[r]);
    }
#pragma unroll
    for (int r = 0; r < kSub; ++r) {
      float kx[DS];
      to_float<T, DS>(raw[r], kx);
      const int j = base + r * NSLOT + slot;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float sc = 0.f;
#pragma unroll
        for (int i = 0; i < DS; ++i) sc = fmaf(qv[g][i], kx[i], sc);
        sc = L == 8 ? octet_sum(sc) : hex_sum(sc);
        if (dl == g && j < n) s_score[g * kMaxPart + j] = blk[r] >= 0 ? sc : -INFINITY;
      }
    }
  }
  // the wave's first value batch is requested before the softmax pass: the workgroups of a CU
  // reach that pass together, and the requests keep the memory pipe busy across it
  Raw<T, DS> vraw[kSub];
  int vblk[kSub];
  auto request_values = [&](int base) {
#pragma unroll
    for (int r = 0; r < kSub; ++r) {
      int off = 0;
      vblk[r] = block_of(base + r * NSLOT + slot, off);
      if (vblk[r] >= 0)
        load_raw<T, DS>(p.v, (int64_t)vblk[r] * p.sv_blk + (int64_t)off * p.sv_tok + (int64_t)kvh * p.sv_head + dl * DS,
                        vraw[r]);
    }
  };
  request_values(wave * kBatch);
  __syncthreads();

  // pass 2: per-head max and exp2, in place (wave w takes heads w, w + 4)
  for (int g = wave; g < G; g += kWaves) {
    float m = -INFINITY;
    for (int j = lane; j < n; j += 64) m = fmaxf(m, s_score[g * kMaxPart + j]);
    m = wave_max(m);
    float l = 0.f;
    for (int j = lane; j < n; j += 64) {
      const float e = m == -INFINITY ? 0.f : exp2f(s_score[g * kMaxPart + j] - m);
      s_score[g * kMaxPart + j] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      s_m[g] = m;
      s_l[g] = l;
    }
  }
  __syncthreads();

  // pass 3: probability-weighted values, the same batches
  float acc[G][DS];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < DS; ++i) acc[g][i] = 0.f;
  for (int base = wave * kBatch; base < n; base += kWaves * kBatch) {
    if (base != wave * kBatch) request_values(base);
#pragma unroll
    for (int r = 0; r < kSub; ++r) {
      if (vblk[r] < 0) continue;
      float vx[DS];
      to_float<T, DS>(vraw[r], vx);
      const int j = base + r * NSLOT + slot;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float w = s_score[g * kMaxPart + j];
#pragma unroll
        for (int i = 0; i < DS; ++i) acc[g][i] = fmaf(w, vx[i], acc[g][i]);
      }
    }
  }
  // sum the position slots of the wave, then the waves through LDS
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < DS; ++i) acc[g][i] = slot_sum<L>(acc[g][i]);
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < DS; ++i) s_red[(wave * G + g) * D + dl * DS + i] = acc[g][i];
  }
  __syncthreads();

  const bool direct = n_parts == 1;
  for (int e = threadIdx.x; e < G * D; e += kThreads) {
    const int g = e / D, d = e % D;
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) o += s_red[(w * G + g) * D + d];
    const int h = kvh * G + g;
    if (direct) {
      const float l = s_l[g];
      store_one<T>(p.out, (int64_t)qi * p.so_tok + (int64_t)h * p.so_head + d, l > 0.f ? o / l : 0.f);
    } else if (p.ws_acc && part < p.max_parts) {
      const int64_t slot_idx = ((int64_t)qi * p.hq + h) * p.max_parts + part;
      st_dev(&p.ws_acc[slot_idx * D + d], o);
      if (d == 0) {
        st_dev(&p.ws_ml[slot_idx * 2], s_m[g]);
        st_dev(&p.ws_ml[slot_idx * 2 + 1], s_l[g]);
      }
    }
  }
  if (direct || !p.ws_acc || part >= p.max_parts) return;

  // Split row: the last of its partitions to arrive merges them (max-rescaled sums, one pass)
  // and resets the row's counter. Every store above completes before the counter moves.
  const int arrivals = n_parts < p.max_parts ? n_parts : p.max_parts;
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int32_t* counter = p.counters + (int64_t)qi * p.hkv + kvh;
  // The partials went out through agent-scope atomic stores (served at the device coherence
  // point, past the per-XCD L2s) completed by the s_waitcnt above, and are read back through
  // agent-scope atomic loads, so the ticket needs no release / acquire fence (a buffer_wbl2 /
  // buffer_inv of the whole L2: 106 -> 128 us at 64 x 2048 decode).
  if (threadIdx.x == 0) s_last = atomicAdd(counter, 1) == arrivals - 1;
  __syncthreads();
  if (!s_last) return;
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (arrivals <= kMaxPart) {
    // weights w_i / L of the partitions into LDS (one wave per head, lanes over partitions), then
    // every output is an independent weighted sum of the partitions' unnormalised outputs
    for (int g = wave; g < G; g += kWaves) {
      const int64_t base = ((int64_t)qi * p.hq + kvh * G + g) * p.max_parts;
      float m = -INFINITY;
      for (int i = lane; i < arrivals; i += 64) m = fmaxf(m, ld_dev(&p.ws_ml[(base + i) * 2]));
      m = wave_max(m);
      float l = 0.f;
      for (int i = lane; i < arrivals; i += 64) {
        const float mi = ld_dev(&p.ws_ml[(base + i) * 2]);
        const float w = (m == -INFINITY || mi == -INFINITY) ? 0.f : exp2f(mi - m);
        s_score[g * kMaxPart + i] = w;
        l = fmaf(w, ld_dev(&p.ws_ml[(base + i) * 2 + 1]), l);
      }
      l = wave_sum(l);
      if (lane == 0) s_l[g] = l;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < G * D; e += kThreads) {
      const int g = e / D, d = e % D;
      const int h = kvh * G + g;
      const int64_t base = ((int64_t)qi * p.hq + h) * p.max_parts;
      float o = 0.f;
#pragma unroll 4
      for (int i = 0; i < arrivals; ++i) o = fmaf(s_score[g * kMaxPart + i], ld_dev(&p.ws_acc[(base + i) * D + d]), o);
      const float l = s_l[g];
      store_one<T>(p.out, (int64_t)qi * p.so_tok + (int64_t)h * p.so_head + d, l > 0.f ? o / l : 0.f);
    }
    return;
  }
  // more partitions than the LDS weight table holds: one pass of max-rescaled sums per output
  for (int e = threadIdx.x; e < G * D; e += kThreads) {
    const int g = e / D, d = e % D;
    const int h = kvh * G + g;
    const int64_t base = ((int64_t)qi * p.hq + h) * p.max_parts;
    float m = -INFINITY, l = 0.f, o = 0.f;
    for (int i = 0; i < arrivals; ++i) {
      const float mi = ld_dev(&p.ws_ml[(base + i) * 2]);
      const float li = ld_dev(&p.ws_ml[(base + i) * 2 + 1]);
      const float ai = ld_dev(&p.ws_acc[(base + i) * D + d]);
      if (mi == -INFINITY) continue;  // a partition whose keys were all skipped
      if (mi > m) {
        const float r = m == -INFINITY ? 0.f : exp2f(m - mi);
        l *= r;
        o *= r;
        m = mi;
      }
      const float w = exp2f(mi - m);
      l = fmaf(w, li, l);
      o = fmaf(w, ai, o);
    }
    store_one<T>(p.out, (int64_t)qi * p.so_tok + (int64_t)h * p.so_head + d, l > 0.f ? o / l : 0.f);
  }
}

// ---- prefill kernel: query tiles on MFMA -------------------------------------------------------
//
// Sequences with several query tokens (chunked prefill) go by query tile: one workgroup of four
// waves per (tile, KV head, KV partition) holds kPfCols = 128 query columns -- kPfCols / G tokens
// of one sequence times the G query heads of the KV head, column c = token (c / G), head (c % G),
// 32 columns per wave -- and walks the partition's positions 64 at a time.  Each step's key and
// value rows are read from memory once for the whole tile (all 256 threads load them into LDS:
// keys as rows, values transposed, dims as rows), so each row is read once per 128 columns
// instead of once per query token.  On v_mfma_f32_32x32x16 (bf16 or f16 operands, float32
// accumulation), per wave:
//   * S^T = K Q^T for the step's two 32-position row blocks: rows positions, columns the wave's
//     queries.  A lane holds one query column (lane % 32) of 16 positions per block, so the
//     online softmax of a column (max, exp2, sum) runs in the lane plus one exchange with
//     lane ^ 32;
//   * O^T += V^T P^T over the step's four 16-position k-steps, the probabilities taken straight
//     from the S^T layout as the B operand: k-slot i of the lanes of half h is position
//     16 s + 8 (i / 4) + 4 h + i % 4 of the step, and the V^T operand is read in that order from
//     the transposed value rows (two 8-byte reads).  P goes in as two 16-bit parts, hi = RN(p)
//     and lo = RN(p - hi): both products with a value are exact in float32, so the sum carries p
//     to about 2^-17 relative, the float32 arithmetic of the reference's kernel (a single 16-bit
//     P would round each weight by up to 2^-9).
// The scores are the float32 dot products times scale * log2(e) and exp2 replaces exp, as in the
// decode kernel.  A tile whose positions span several partitions has them merged by the last to
// arrive, as the decode kernel's split rows are.

constexpr int kPfWaves = 4;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfCols = 32 * kPfWaves;   // query columns of a tile (32 per wave)
constexpr int kPfPos = 64;               // positions per step (two 32-row blocks)
constexpr int kPfMaxPart = 1024;
constexpr int kPfMinPart = 256;
constexpr int kPfTargetGroups = 512;     // two four-wave workgroups per CU
static_assert(kPfCols == NS_PA_TILE_COLUMNS, "the header's tile width");

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// The MFMA and the 16-bit type's conversions: pack2 rounds two floats to nearest even into one
// word (low half the first; v_cvt_pk_bf16_f32 for bfloat16), lo / hi widen a word's halves back.
template <typename T> struct Mma;
template <> struct Mma<Bf16> {
  typedef bf16x8_t vec;
  static __device__ __forceinline__ f32x16_t mma(vec a, vec b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2_t));
  }
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
};
template <> struct Mma<F16> {
  typedef f16x8_t vec;
  static __device__ __forceinline__ f32x16_t mma(vec a, vec b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2_t));
  }
  static __device__ __forceinline__ float lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)w); }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
};

struct PfParams {
  const int32_t* tiles;   // (n_tiles, 3): sequence, first query token (flat index), token count
  float* ws_acc;          // (n_tiles, hkv, max_parts, kPfCols, D) unnormalised partition outputs
  float* ws_ml;           // (n_tiles, hkv, max_parts, kPfCols, 2) partition max (log2 units), sum
  int32_t* counters;      // (n_tiles, hkv) arrivals of split tiles; zero between calls
  int32_t part_tokens;    // positions per partition (a multiple of kPfPos)
  int32_t max_parts;      // at least 1
};

template <typename T, int D, int G>
__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void pa_prefill_kernel(PaParams p,
                                                                                                        PfParams f) {
  using M = Mma<T>;
  using vec = typename M::vec;
  constexpr int BQ = kPfCols / G;                 // tokens per tile
  constexpr int KS = D / 16;                      // k-steps of S^T = K Q^T
  constexpr int DB = D / 32;                      // 32-dim blocks of O^T
  constexpr int CPP = D / 8;                      // 16-byte chunks of a key or value row
  constexpr int LPT = kPfPos * CPP / kPfThreads;  // chunks of each kind a thread loads per step
  constexpr int PK = D * 2 + 16;                  // bytes per staged key or value row
  static_assert(LPT * kPfThreads == kPfPos * CPP, "the step's chunks split evenly over the threads");
  __shared__ __align__(16) unsigned char s_k[kPfPos * PK];
  __shared__ __align__(16) unsigned char s_v[kPfPos * PK];
  __shared__ __align__(16) uint8_t s_ok[kPfPos];
  __shared__ int s_blk[kPfMaxPart + 2];
  __shared__ int s_last;

  const int tile = blockIdx.x, kvh = blockIdx.y, part = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5, c32 = lane & 31;
  const int seq = f.tiles[3 * tile];
  const int t0 = f.tiles[3 * tile + 1];
  const int nq = f.tiles[3 * tile + 2];
  // a tile must hold 1 .. BQ consecutive query tokens of one sequence: anything else is flagged
  // and left alone (nothing is read or written out of bounds)
  if (seq < 0 || seq >= p.num_seqs || nq < 1 || nq > BQ || t0 < p.qsl[seq] || t0 + nq > p.qsl[seq] + p.qlens[seq] ||
      t0 + nq > p.total_q) {
    if (tid == 0 && part == 0 && p.status) atomicOr(p.status, NS_PA_STATUS_BAD_TILE);
    return;
  }
  const int seq_len = p.seq_lens[seq];
  const int kv_pos0 = seq_len - p.qlens[seq] + (t0 - p.qsl[seq]);   // the first token's KV position
  int lt = kv_pos0 + nq < seq_len ? kv_pos0 + nq : seq_len;          // positions the last token sees
  if (lt < 0) lt = 0;
  const int n_parts = (lt + f.part_tokens - 1) / f.part_tokens;
  if (part == 0 && n_parts > f.max_parts && tid == 0 && p.status) atomicOr(p.status, NS_PA_STATUS_SEQ_TOO_LONG);

  // the lane's column: token tok, head hd, visible positions kvl (-1: a padding column, never written)
  const int c = wave * 32 + c32;
  const int tok = c / G, hd = c % G;
  int kvl = -1;
  if (c < BQ * G && tok < nq) {
    const int kl = kv_pos0 + tok + 1 < seq_len ? kv_pos0 + tok + 1 : seq_len;
    kvl = kl > 0 ? kl : 0;
  }
  const int64_t obase = (int64_t)(t0 + tok) * p.so_tok + (int64_t)(kvh * G + hd) * p.so_head;
  if (part >= n_parts) {
    if (part == 0 && kvl >= 0 && h == 0)   // no visible key for any token of the tile: zeros
      for (int d = 0; d < D; ++d) store_one<T>(p.out, obase + d, 0.f);
    return;
  }
  const int j0 = part * f.part_tokens;
  const int j1 = lt < j0 + f.part_tokens ? lt : j0 + f.part_tokens;
  const int kend = kvl < j1 ? kvl : j1;   // the column's positions below kend are visible here
  // the smallest kend of the wave's columns (padding columns aside): positions below it are
  // visible to every column of the wave
  int kend_w = kvl >= 0 ? kend : INT32_MAX;
#pragma unroll
  for (int sh = 1; sh < 64; sh <<= 1) kend_w = min(kend_w, __shfl_xor(kend_w, sh));
  const int32_t* bt_row = p.bt + (int64_t)seq * p.sbt;
  // the partition's slice of the block table, validated once, into LDS
  const int bi0 = j0 / p.block_size;
  const int nbi = (j1 - 1) / p.block_size - bi0 + 1;
  int bad = 0;
  for (int i = tid; i < nbi; i += kPfThreads) {
    const int bi = bi0 + i;
    int blk = bi < p.max_blocks_per_seq ? bt_row[bi] : -1;
    if (blk < 0 || blk >= p.num_blocks) {
      blk = -1;
      bad = 1;
      if (p.status) atomicOr(p.status, NS_PA_STATUS_BAD_BLOCK);
    }
    s_blk[i] = blk;
  }

  // Q^T operand: column c, dims 16 ks + 8 h .. + 7 (zeros for a padding column)
  vec qop[KS];
  {
    const int64_t qoff = (int64_t)(t0 + tok) * p.sq_tok + (int64_t)(kvh * G + hd) * p.sq_head;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (kvl >= 0) w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(p.q) + (qoff + 16 * ks + 8 * h) * 2);
      qop[ks] = __builtin_bit_cast(vec, w);
    }
  }
  // the slice, and whether any of its blocks is invalid (then every step masks by position)
  const bool any_bad = __syncthreads_or(bad) != 0;

  // the step's key and value rows: chunk i = tid + kPfThreads r is position i / CPP, dims
  // 8 (i % CPP) .. + 7; zeros past the partition or for an invalid block
  // every chunk of the thread has dims 8 dc .. (kPfThreads is a multiple of CPP); the host
  // keeps token strides times block_size below 2^31, so a slot's offset is a 32-bit product
  const int dc0 = tid % CPP;
  const char* kbase = reinterpret_cast<const char*>(p.k) + ((int64_t)kvh * p.sk_head + 8 * dc0) * 2;
  const char* vbase = reinterpret_cast<const char*>(p.v) + ((int64_t)kvh * p.sv_head + 8 * dc0) * 2;
  const int sk_tok = (int)p.sk_tok, sv_tok = (int)p.sv_tok;
  auto load_step = [&](int jt, u32x4 (&kreg)[LPT], u32x4 (&vreg)[LPT], bool (&okr)[LPT]) {
#pragma unroll
    for (int r = 0; r < LPT; ++r) {
      const int j = jt + (tid + kPfThreads * r) / CPP;
      int blk = -1, off = 0;
      if (j < j1) {
        int bi;
        if (p.bs_shift >= 0) { bi = j >> p.bs_shift; off = j & (p.block_size - 1); }
        else { bi = j / p.block_size; off = j - bi * p.block_size; }
        blk = s_blk[bi - bi0];
      }
      okr[r] = blk >= 0;
      kreg[r] = u32x4{0u, 0u, 0u, 0u};
      vreg[r] = u32x4{0u, 0u, 0u, 0u};
      if (blk >= 0) {
        kreg[r] = *reinterpret_cast<const u32x4*>(kbase + ((int64_t)blk * p.sk_blk + off * sk_tok) * 2);
        vreg[r] = *reinterpret_cast<const u32x4*>(vbase + ((int64_t)blk * p.sv_blk + off * sv_tok) * 2);
      }
    }
  };
  auto store_step = [&](const u32x4 (&kreg)[LPT], const u32x4 (&vreg)[LPT], const bool (&okr)[LPT]) {
#pragma unroll
    for (int r = 0; r < LPT; ++r) {
      const int i = tid + kPfThreads * r;
      const int pos = i / CPP, dc = i % CPP;
      *reinterpret_cast<u32x4*>(s_k + pos * PK + dc * 16) = kreg[r];
      *reinterpret_cast<u32x4*>(s_v + pos * PK + dc * 16) = vreg[r];
      if (dc == 0) s_ok[pos] = okr[r] ? 1 : 0;
    }
  };

  f32x16_t acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[db][e] = 0.f;
  float m = -INFINITY, l = 0.f;

  // The transposing read (ds_read_b64_tr_b16): in each 16-lane group, lane j's four results are
  // element j % 4 of the 4-element rows that lanes 4 m + j / 4 address, m = 0..3.  So that lane L
  // receives positions 16 s + 4 h + m of dim 32 db + L % 32, lane L addresses position
  // 16 s + 4 (L / 32) + (L % 16) / 4, dims 32 db + 16 ((L / 16) % 2) + 4 (L % 4) .. + 3.
  const int tr_pos = 4 * (lane >> 5) + ((lane & 15) >> 2);
  const int tr_dim = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  u32x4 kreg[LPT], vreg[LPT];
  bool okr[LPT];
  load_step(j0, kreg, vreg, okr);
  for (int jt = j0; jt < j1; jt += kPfPos) {
    __syncthreads();   // the previous step's reads of the staged rows are done
    store_step(kreg, vreg, okr);
    __syncthreads();   // this step's rows staged
    // the next step's rows, in flight across this step's products and softmax
    if (jt + kPfPos < j1) load_step(jt + kPfPos, kreg, vreg, okr);
    // S^T = K Q^T for the step's two 32-position row blocks (two independent MFMA chains)
    f32x16_t st[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int e = 0; e < 16; ++e) st[rb][e] = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(s_k + (32 * rb + c32) * PK + (16 * ks + 8 * h) * 2);
        st[rb] = M::mma(__builtin_bit_cast(vec, w), qop[ks], st[rb]);
      }
    }
    // the online softmax of the lane's column over the step's 64 positions (element e of block
    // rb: position 32 rb + 8 (e / 4) + 4 h + e % 4; the other half in lane ^ 32)
    float mt = -INFINITY;
    if (jt + kPfPos <= kend_w && !any_bad) {   // every position of the step visible to every column
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          st[rb][e] *= p.scale_log2;
          mt = fmaxf(mt, st[rb][e]);
        }
    } else {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        uint32_t okw[4] = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
        if (any_bad) {
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) okw[q4] = *reinterpret_cast<const uint32_t*>(s_ok + 32 * rb + 8 * q4 + 4 * h);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = 32 * rb + 8 * (e >> 2) + 4 * h + (e & 3);
          const bool ok = jt + r < kend && ((okw[e >> 2] >> (8 * (e & 3))) & 0xffu) != 0u;
          st[rb][e] = ok ? st[rb][e] * p.scale_log2 : -INFINITY;
          mt = fmaxf(mt, st[rb][e]);
        }
      }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    // The column's reference m moves only when a score exceeds it by more than 8 (log2 units),
    // to the new maximum: weights stay at most 2^8 and the accumulators are rescaled rarely.
    // exp2 by v_exp_f32 (a weight below 2^-126 flushes to zero); -inf scores weigh 0, and a
    // column with no score yet subtracts 0.
    const bool move = mt > m + 8.f;
    const float mn = move ? mt : m;
    const float msub = mn == -INFINITY ? 0.f : mn;
    const float alpha = move ? __builtin_amdgcn_exp2f(m - msub) : 1.f;
    m = mn;
    if (__ballot(move) != 0ull) {   // a column's reference moved: rescale
      l *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[db][e] *= alpha;
    }
    // per 16-position k-step s: P as the hi / lo B operands, then O^T += V^T P^T with the V^T
    // operand of dim 32 db + c32 (k-slot i of half h at position 16 s + 8 (i / 4) + 4 h + i % 4)
    // read from the value rows by two transposing reads (k-slots 0-3, then 4-7)
    float ls = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4 wh, wl;
#pragma unroll
      for (int i2 = 0; i2 < 4; ++i2) {
        const float p0 = __builtin_amdgcn_exp2f(st[s >> 1][8 * (s & 1) + 2 * i2] - msub);
        const float p1 = __builtin_amdgcn_exp2f(st[s >> 1][8 * (s & 1) + 2 * i2 + 1] - msub);
        ls += p0 + p1;
        wh[i2] = M::pack2(p0, p1);
        wl[i2] = M::pack2(p0 - M::lo(wh[i2]), p1 - M::hi(wh[i2]));
      }
      const vec phi = __builtin_bit_cast(vec, wh), plo = __builtin_bit_cast(vec, wl);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const unsigned char* src = s_v + (16 * s + tr_pos) * PK + (32 * db + tr_dim) * 2;
        const u32x2 lo4 = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                        (__attribute__((address_space(3))) i16x4*)(src)));
        const u32x2 hi4 = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                        (__attribute__((address_space(3))) i16x4*)(src + 8 * PK)));
        const u32x4 w = {lo4[0], lo4[1], hi4[0], hi4[1]};
        const vec a = __builtin_bit_cast(vec, w);
        acc[db] = M::mma(a, phi, acc[db]);
        acc[db] = M::mma(a, plo, acc[db]);
      }
    }
    ls += __shfl_xor(ls, 32);
    l += ls;
  }

  // O^T layout: lane l, element e -> column c, dim 32 db + 8 (e / 4) + 4 h + e % 4
  const bool direct = n_parts == 1;
  const int64_t wbase = ((int64_t)tile * p.hkv + kvh) * f.max_parts;
  if ((direct || part < f.max_parts) && kvl >= 0) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int d = 32 * db + 8 * (e >> 2) + 4 * h + (e & 3);
        if (direct) store_one<T>(p.out, obase + d, l > 0.f ? acc[db][e] / l : 0.f);
        else st_dev(&f.ws_acc[((wbase + part) * kPfCols + c) * D + d], acc[db][e]);
      }
    if (!direct && h == 0) {
      st_dev(&f.ws_ml[((wbase + part) * kPfCols + c) * 2], m);
      st_dev(&f.ws_ml[((wbase + part) * kPfCols + c) * 2 + 1], l);
    }
  }
  if (direct || part >= f.max_parts) return;

  // split tile: the last partition to arrive merges (the partials crossed through agent-scope
  // atomic stores completed by the s_waitcnt, read back through agent-scope loads)
  const int arrivals = n_parts < f.max_parts ? n_parts : f.max_parts;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int32_t* counter = f.counters + (int64_t)tile * p.hkv + kvh;
  if (tid == 0) s_last = atomicAdd(counter, 1) == arrivals - 1;
  __syncthreads();
  if (!s_last) return;
  if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // The weights w_i = exp2(m_i - max) of every column's partitions and their sum L: up to
  // kPfMergeLds partitions in LDS (the staged key rows are free now), computed once, with all
  // the (m, l) loads of a thread in flight together; then two threads per column, half the dims
  // each, accumulate the partials partition by partition, all of a partition's loads issued
  // before the first is used.
  constexpr int HD = D / 2;
  constexpr int kPfMergeLds = (kPfPos * PK) / (kPfCols * 4) >= 32 ? 32 : 16;   // partitions in the table
  float* s_w = reinterpret_cast<float*>(s_k);        // [i][column] weights
  float* s_L = reinterpret_cast<float*>(s_v);        // [column] the weights' sum of l
  static_assert(kPfMergeLds * kPfCols * 4 <= kPfPos * PK && kPfCols * 4 <= kPfPos * PK, "merge tables fit");
  const int mc = tid >> 1, d0 = (tid & 1) * HD;
  const int ti = mc / G, hg = mc % G;
  const bool live = mc < BQ * G && ti < nq;
  if (arrivals <= kPfMergeLds) {
    if (tid < kPfCols) {
      float mi[kPfMergeLds], li[kPfMergeLds];
#pragma unroll
      for (int i = 0; i < kPfMergeLds; ++i) {
        mi[i] = -INFINITY;
        li[i] = 0.f;
        if (i < arrivals) {
          mi[i] = ld_dev(&f.ws_ml[((wbase + i) * kPfCols + tid) * 2]);
          li[i] = ld_dev(&f.ws_ml[((wbase + i) * kPfCols + tid) * 2 + 1]);
        }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < kPfMergeLds; ++i) mx = fmaxf(mx, mi[i]);
      float L = 0.f;
#pragma unroll
      for (int i = 0; i < kPfMergeLds; ++i) {
        // a partition whose keys were all skipped (m = -inf) weighs 0
        const float w = mi[i] == -INFINITY ? 0.f : exp2f(mi[i] - mx);
        L = fmaf(w, li[i], L);
        if (i < arrivals) s_w[i * kPfCols + tid] = w;
      }
      s_L[tid] = L;
    }
    __syncthreads();
    if (!live) return;
    float o[HD];
#pragma unroll
    for (int d = 0; d < HD; ++d) o[d] = 0.f;
    for (int i = 0; i < arrivals; ++i) {
      const float w = s_w[i * kPfCols + mc];
      const float* src = &f.ws_acc[((wbase + i) * kPfCols + mc) * D + d0];
      float a[HD];
#pragma unroll
      for (int d = 0; d < HD; ++d) a[d] = ld_dev(src + d);
#pragma unroll
      for (int d = 0; d < HD; ++d) o[d] = fmaf(w, a[d], o[d]);
    }
    const float L = s_L[mc];
    const int64_t ob = (int64_t)(t0 + ti) * p.so_tok + (int64_t)(kvh * G + hg) * p.so_head + d0;
#pragma unroll
    for (int d = 0; d < HD; ++d) store_one<T>(p.out, ob + d, L > 0.f ? o[d] / L : 0.f);
    return;
  }
  // more partitions than the LDS table holds: one pass of max-rescaled sums per thread
  if (!live) return;
  float mm = -INFINITY, L = 0.f;
  float o[HD];
#pragma unroll
  for (int d = 0; d < HD; ++d) o[d] = 0.f;
  for (int i = 0; i < arrivals; ++i) {
    const float mi = ld_dev(&f.ws_ml[((wbase + i) * kPfCols + mc) * 2]);
    const float li = ld_dev(&f.ws_ml[((wbase + i) * kPfCols + mc) * 2 + 1]);
    if (mi == -INFINITY) continue;
    const float* src = &f.ws_acc[((wbase + i) * kPfCols + mc) * D + d0];
    float a[HD];
#pragma unroll
    for (int d = 0; d < HD; ++d) a[d] = ld_dev(src + d);
    if (mi > mm) {
      const float r = mm == -INFINITY ? 0.f : exp2f(mm - mi);
      L *= r;
#pragma unroll
      for (int d = 0; d < HD; ++d) o[d] *= r;
      mm = mi;
    }
    const float w = exp2f(mi - mm);
    L = fmaf(w, li, L);
#pragma unroll
    for (int d = 0; d < HD; ++d) o[d] = fmaf(w, a[d], o[d]);
  }
  const int64_t ob = (int64_t)(t0 + ti) * p.so_tok + (int64_t)(kvh * G + hg) * p.so_head + d0;
#pragma unroll
  for (int d = 0; d < HD; ++d) store_one<T>(p.out, ob + d, L > 0.f ? o[d] / L : 0.f);
}

// ---- host side ---------------------------------------------------------------------------------

int pf_part_tokens_for(int32_t n_tiles, int32_t hkv, int32_t max_seq_len) {
  int part = kPfMaxPart;
  while (part > kPfMinPart) {
    const int64_t parts = ((int64_t)max_seq_len + part - 1) / part;
    if ((int64_t)n_tiles * hkv * parts >= kPfTargetGroups) break;
    part >>= 1;
  }
  return part;
}

// Bytes of the prefill tiles' partials (0 when every tile fits one partition).
uint64_t pf_workspace_bytes(int32_t n_tiles, int32_t hkv, int32_t head_dim, int32_t max_seq_len) {
  if (n_tiles <= 0) return 0;
  const int part = pf_part_tokens_for(n_tiles, hkv, max_seq_len);
  const int64_t max_parts = ((int64_t)max_seq_len + part - 1) / part;
  if (max_parts <= 1) return 0;
  return (uint64_t)n_tiles * hkv * max_parts * kPfCols * (head_dim + 2) * sizeof(float);
}

int part_tokens_for(int32_t total_q, int32_t hkv, int32_t max_seq_len) {
  int part = kMaxPart;
  while (part > kMinPart) {
    const int64_t parts = ((int64_t)max_seq_len + part - 1) / part;
    if ((int64_t)total_q * hkv * parts >= kTargetGroups) break;
    part >>= 1;
  }
  return part;
}

int check_sizes(int32_t total_q, int32_t hq, int32_t hkv, int32_t head_dim, int32_t max_seq_len) {
  if (total_q < 0) return fail("total_q must be >= 0 (got %d)", total_q);
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0)
    return fail("num_heads_q (%d) must be a positive multiple of num_kv_heads (%d)", hq, hkv);
  const int g = hq / hkv;
  if (g != 1 && g != 2 && g != 3 && g != 4 && g != 8)
    return fail("query heads per KV head must be 1, 2, 3, 4 or 8 (got %d)", g);
  if (head_dim != 64 && head_dim != 128) return fail("head_dim must be 64 or 128 (got %d)", head_dim);
  if (max_seq_len < 0) return fail("max_seq_len must be >= 0 (got %d)", max_seq_len);
  if (hkv > 65535 || hq > 65535) return fail("too many heads (grid y is at most 65535)");
  return 0;
}

// Bytes of the per-token kernel's partials: total_q query slots (the kernel indexes them by query
// token), the partition length sized for the n_tokens workgroups along x.
uint64_t workspace_bytes(int32_t total_q, int32_t hq, int32_t hkv, int32_t head_dim, int32_t max_seq_len,
                         int32_t n_tokens) {
  const int part = part_tokens_for(n_tokens, hkv, max_seq_len);
  const int64_t max_parts = ((int64_t)max_seq_len + part - 1) / part;
  if (max_parts <= 1) return 0;
  return (uint64_t)total_q * hq * max_parts * (head_dim + 2) * sizeof(float);
}
uint64_t workspace_bytes(int32_t total_q, int32_t hq, int32_t hkv, int32_t head_dim, int32_t max_seq_len) {
  return workspace_bytes(total_q, hq, hkv, head_dim, max_seq_len, total_q);
}

// n_tokens decode workgroups along x (p.tokens or the first n_tokens tokens); the prefill tiles
// when f.tiles is set (16-bit types only)
template <typename T, int D, int G>
void launch(const PaParams& p, const PfParams& f, int n_tokens, int n_tiles, hipStream_t stream) {
  if (n_tokens > 0) {
    dim3 grid(n_tokens, p.hkv, p.max_parts > 0 ? p.max_parts : 1);
    hipLaunchKernelGGL((pa_partition_kernel<T, D, G>), grid, dim3(kThreads), 0, stream, p);
  }
  if constexpr (Elem<T>::bytes == 2) {
    if (n_tiles > 0) {
      dim3 grid(n_tiles, p.hkv, f.max_parts);
      hipLaunchKernelGGL((pa_prefill_kernel<T, D, G>), grid, dim3(kPfThreads), 0, stream, p, f);
    }
  }
}

template <typename T, int D>
void launch_g(const PaParams& p, const PfParams& f, int n_tokens, int n_tiles, int g, hipStream_t stream) {
  switch (g) {
    case 1: launch<T, D, 1>(p, f, n_tokens, n_tiles, stream); break;
    case 2: launch<T, D, 2>(p, f, n_tokens, n_tiles, stream); break;
    case 3: launch<T, D, 3>(p, f, n_tokens, n_tiles, stream); break;
    case 4: launch<T, D, 4>(p, f, n_tokens, n_tiles, stream); break;
    default: launch<T, D, 8>(p, f, n_tokens, n_tiles, stream); break;
  }
}

template <typename T>
void launch_d(const PaParams& p, const PfParams& f, int n_tokens, int n_tiles, int d, int g, hipStream_t stream) {
  if (d == 64) launch_g<T, 64>(p, f, n_tokens, n_tiles, g, stream);
  else launch_g<T, 128>(p, f, n_tokens, n_tiles, g, stream);
}

}  // namespace

extern "C" {

int ns_pa_abi_version(void) { return NS_PA_ABI_VERSION; }

const char* ns_pa_last_error(void) { return g_err; }

int ns_paged_attention_workspace_bytes(int32_t total_q, int32_t num_heads_q, int32_t num_kv_heads,
                                       int32_t head_dim, int32_t max_seq_len, uint64_t* bytes) {
  if (!bytes) return fail("bytes is NULL");
  if (check_sizes(total_q, num_heads_q, num_kv_heads, head_dim, max_seq_len)) return 1;
  *bytes = workspace_bytes(total_q, num_heads_q, num_kv_heads, head_dim, max_seq_len);
  return 0;
}

int ns_paged_attention_call_workspace(const ns_paged_attn_args* a, uint64_t* bytes, uint64_t* counters) {
  if (!a || !bytes || !counters) return fail("a pointer argument is NULL");
  if (check_sizes(a->total_q, a->num_heads_q, a->num_kv_heads, a->head_dim, a->max_seq_len)) return 1;
  if (a->n_decode_tokens < 0 || a->n_prefill_tiles < 0) return fail("token and tile counts must be >= 0");
  const int32_t n_tokens = a->decode_tokens ? a->n_decode_tokens : a->total_q;
  const uint64_t dec =
      workspace_bytes(a->total_q, a->num_heads_q, a->num_kv_heads, a->head_dim, a->max_seq_len, n_tokens);
  const int32_t tiles = a->prefill_tiles ? a->n_prefill_tiles : 0;
  *bytes = dec + pf_workspace_bytes(tiles, a->num_kv_heads, a->head_dim, a->max_seq_len);
  *counters = (uint64_t)a->total_q * a->num_kv_heads + (uint64_t)tiles * a->num_kv_heads;
  return 0;
}

int ns_paged_attention(const ns_paged_attn_args* a, hipStream_t stream) {
  if (!a) return fail("args is NULL");
  if (check_sizes(a->total_q, a->num_heads_q, a->num_kv_heads, a->head_dim, a->max_seq_len)) return 1;
  if (a->dtype != NS_PA_DTYPE_F32 && a->dtype != NS_PA_DTYPE_BF16 && a->dtype != NS_PA_DTYPE_F16)
    return fail("dtype must be NS_PA_DTYPE_F32, _BF16 or _F16 (got %d)", a->dtype);
  if (a->total_q == 0) return 0;
  if (a->num_seqs <= 0) return fail("num_seqs must be > 0 when total_q > 0 (got %d)", a->num_seqs);
  if (a->block_size <= 0) return fail("block_size must be > 0 (got %d)", a->block_size);
  if (a->num_blocks <= 0) return fail("num_blocks must be > 0 (got %d)", a->num_blocks);
  if (!a->query || !a->k_cache || !a->v_cache || !a->out || !a->block_tables || !a->seq_lens ||
      !a->query_start_loc || !a->query_lens)
    return fail("a tensor pointer is NULL");
  const int esz = a->dtype == NS_PA_DTYPE_F32 ? 4 : 2;
  // 16-byte vector loads of each lane's head_dim/8 slice: rows and strides 16-byte aligned
  const int64_t strides[] = {a->stride_q_token, a->stride_q_head, a->stride_k_block, a->stride_k_token,
                             a->stride_k_head, a->stride_v_block, a->stride_v_token, a->stride_v_head};
  for (int64_t s : strides)
    if ((s * esz) % 16 != 0) return fail("query/cache strides must be multiples of 16 bytes");
  if (((uintptr_t)a->query | (uintptr_t)a->k_cache | (uintptr_t)a->v_cache) % 16 != 0)
    return fail("query and cache pointers must be 16-byte aligned");
  if (a->stride_bt_seq < 0) return fail("stride_bt_seq must be >= 0");
  if (a->stride_k_token < 0 || a->stride_v_token < 0 ||
      (int64_t)a->block_size * (a->stride_k_token > a->stride_v_token ? a->stride_k_token : a->stride_v_token) >=
          ((int64_t)1 << 31))
    return fail("token strides times block_size must lie in [0, 2^31)");
  if (a->max_blocks_per_seq < 0) return fail("max_blocks_per_seq must be >= 0");
  // the prefill tiles (16-bit types) and the token list of the per-token kernel
  if (a->n_decode_tokens < 0 || a->n_prefill_tiles < 0) return fail("token and tile counts must be >= 0");
  if (a->prefill_tiles && a->dtype == NS_PA_DTYPE_F32)
    return fail("prefill tiles take bfloat16 or float16 (float32 queries go through the per-token kernel)");
  if (a->prefill_tiles && !a->decode_tokens)
    return fail("a call with prefill tiles lists its other query tokens in decode_tokens");
  const int32_t n_tiles = a->prefill_tiles ? a->n_prefill_tiles : 0;
  const int32_t n_tokens = a->decode_tokens ? a->n_decode_tokens : a->total_q;
  const uint64_t need =
      workspace_bytes(a->total_q, a->num_heads_q, a->num_kv_heads, a->head_dim, a->max_seq_len, n_tokens);
  if (need > 0 && !a->counters) return fail("a call with split rows needs the zero-filled counters buffer");
  const int part = part_tokens_for(n_tokens, a->num_kv_heads, a->max_seq_len);
  const int64_t max_parts = ((int64_t)a->max_seq_len + part - 1) / part;
  if (max_parts > 65535) return fail("max_seq_len too large");
  const uint64_t pf_need = pf_workspace_bytes(n_tiles, a->num_kv_heads, a->head_dim, a->max_seq_len);
  if (need + pf_need > 0 && (!a->workspace || a->workspace_bytes < need + pf_need))
    return fail("workspace of %llu bytes needed (got %llu)", (unsigned long long)(need + pf_need),
                (unsigned long long)a->workspace_bytes);
  if (pf_need > 0 && !a->counters) return fail("a call with split tiles needs the zero-filled counters buffer");
  const int pf_part = pf_part_tokens_for(n_tiles, a->num_kv_heads, a->max_seq_len);
  const int64_t pf_max_parts = ((int64_t)a->max_seq_len + pf_part - 1) / pf_part;
  if (pf_max_parts > 65535) return fail("max_seq_len too large");

  PaParams p;
  p.q = a->query;
  p.k = a->k_cache;
  p.v = a->v_cache;
  p.out = a->out;
  p.bt = a->block_tables;
  p.seq_lens = a->seq_lens;
  p.qsl = a->query_start_loc;
  p.qlens = a->query_lens;
  p.status = a->status;
  p.ws_acc = reinterpret_cast<float*>(a->workspace);
  p.ws_ml = need ? p.ws_acc + (uint64_t)a->total_q * a->num_heads_q * max_parts * a->head_dim : nullptr;
  p.counters = a->counters;
  p.sq_tok = a->stride_q_token;
  p.sq_head = a->stride_q_head;
  p.sk_blk = a->stride_k_block;
  p.sk_tok = a->stride_k_token;
  p.sk_head = a->stride_k_head;
  p.sv_blk = a->stride_v_block;
  p.sv_tok = a->stride_v_token;
  p.sv_head = a->stride_v_head;
  p.so_tok = a->stride_o_token;
  p.so_head = a->stride_o_head;
  p.sbt = a->stride_bt_seq;
  p.num_seqs = a->num_seqs;
  p.hq = a->num_heads_q;
  p.hkv = a->num_kv_heads;
  p.block_size = a->block_size;
  p.bs_shift = -1;
  if ((a->block_size & (a->block_size - 1)) == 0)
    for (int sh = 0; sh < 31; ++sh)
      if ((1 << sh) == a->block_size) p.bs_shift = sh;
  p.num_blocks = a->num_blocks;
  p.max_blocks_per_seq = a->max_blocks_per_seq;
  p.part_tokens = part;
  p.max_parts = (int32_t)max_parts;
  p.scale_log2 = a->scale * kLog2e;
  p.total_q = a->total_q;
  p.tokens = a->decode_tokens;

  PfParams f;
  f.tiles = a->prefill_tiles;
  char* ws = reinterpret_cast<char*>(a->workspace);
  f.ws_acc = pf_need ? reinterpret_cast<float*>(ws + need) : nullptr;
  f.ws_ml = pf_need ? f.ws_acc + (uint64_t)n_tiles * a->num_kv_heads * pf_max_parts * kPfCols * a->head_dim : nullptr;
  f.counters = a->counters ? a->counters + (int64_t)a->total_q * a->num_kv_heads : nullptr;
  f.part_tokens = pf_part;
  f.max_parts = pf_max_parts > 0 ? (int32_t)pf_max_parts : 1;

  const int g = a->num_heads_q / a->num_kv_heads;
  switch (a->dtype) {
    case NS_PA_DTYPE_F32: launch_d<float>(p, f, n_tokens, 0, a->head_dim, g, stream); break;
    case NS_PA_DTYPE_BF16: launch_d<Bf16>(p, f, n_tokens, n_tiles, a->head_dim, g, stream); break;
    default: launch_d<F16>(p, f, n_tokens, n_tiles, a->head_dim, g, stream); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("kernel launch failed: %s", hipGetErrorString(e));
  return 0;
}

}  // extern "C"
