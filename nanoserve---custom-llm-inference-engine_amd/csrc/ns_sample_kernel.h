// gfx950 token-sampler kernel: one 1024-thread workgroup per sampled row.
//
// Replaces the op sequence of nanoserve/scheduler/sampler.py:28-89 for one row:
// repetition penalty (:31-38), temperature (:40-51), top-k (:53-58), top-p
// (:60-73), softmax and the NaN guard (:75-80), greedy argmax (:82-83) and the
// draw (:84-89, inverse CDF against a caller-supplied uniform).
//
// Work split inside the workgroup
//   waves 0..14 ("row threads", RT = 960) own the row's 16-byte chunks:
//     chunk c belongs to thread c % RT, slot c / RT (coalesced uint4 loads);
//   wave 15 ("history wave") owns the extras list: the row's unique penalty
//     history ids with their penalized values, plus the < 8 tail elements that
//     do not fill a whole chunk.  History positions are set to -inf in the
//     chunk layout (via an LDS presence bitmap), so every statistic is the
//     chunk-layout statistic combined with the extras statistic.
//
// Passes
//   P1 (the only HBM pass for greedy and top-k rows): stream the row, mask
//      history positions, row max (NaN-propagating), first argmax chunk, and
//      8 group maxima per thread (group = a run of consecutive chunk rows).
//   top-k (k <= 1024): a threshold tau with count(x >= tau) >= k is read off a
//      linear-bin histogram of the group maxima; the chunks of groups whose
//      maximum reaches tau are re-read (L2 / Infinity Cache hits), elements
//      >= tau are compacted into LDS and the exact k-th largest, top-p cut,
//      softmax and draw are done there (bitonic sorts in LDS).
//   other rows: histogram passes over re-read data (L2 / Infinity Cache):
//      count histogram for large k, fixed-point mass histogram for top-p,
//      per-chunk-row mass sums for the inverse-CDF draw.
#pragma once

#include "ns_device.h"

namespace ns {

constexpr int RT = NT - 64;      // row threads (waves 0..14)
constexpr int CAP = 4096;        // LDS candidate capacity
constexpr int NB = 2048;         // histogram bins
constexpr int KSMALL = 1024;     // largest k handled by the chunk-maxima threshold
constexpr int HPT = 8;           // history ids per thread held in registers (one batch of 8192)
constexpr int GATHER = 2;        // history-value gathers in flight per history-wave lane
constexpr int LDS_HIST = HPT * NT;   // longest history whose unique ids the general code keeps in LDS
constexpr int MAX_HIST = 1 << 20;    // per-row history limit (longer ids stream in batches)
constexpr int NGROUP = 8;        // streaming mode: chunk-maxima groups per thread
constexpr int MAX_LEVELS = 4;    // histogram refinement rounds
constexpr int INFO_WORDS = 8;

enum : int32_t {
  PATH_GREEDY = 1, PATH_UNIFORM = 2, PATH_TOPK_SET = 3, PATH_GENERIC_SET = 4, PATH_LARGE_DRAW = 5,
  PATH_ERROR = 9
};
enum : int32_t {
  FLAG_BAD_HIST_ID = 1, FLAG_HIST_TOO_LONG = 2, FLAG_BAD_ROW = 4, FLAG_CAND_OVERFLOW = 8,
  FLAG_REFINE_LIMIT = 16, FLAG_LOCATE_FALLBACK = 32
};

struct KParams {
  const void* logits;
  int64_t row_stride;      // elements
  int64_t vocab;
  int64_t n_rows_total;
  const int64_t* sample_idx;
  const float* temperature;
  const int32_t* top_k;
  const float* top_p;
  const float* penalty;
  const float* pen_rcp;   // [B] RN(1/p) per row: the penalty's positive branch as x * pen_rcp[row]
                          // (NS_PENALTY_RECIPROCAL), or NULL: the division
  const int32_t* hist_off;
  const int32_t* hist_ids;
  const int32_t* hist_slot;   // device-resident histories: request slot of each row (-1: none), or NULL
  const int32_t* hist_len;    // slot lengths (hist_ids then holds hist_nslots * hist_cap ids)
  int32_t hist_nslots, hist_cap;
  const float* uniforms;
  IdSink out_ids;
  float* out_probs;
  int32_t* out_info;
  const int32_t* status;   // [n_sample] from the segment kernel (0 = resolved there), or NULL: every row
  int32_t n_sample;
  int32_t fast;            // 1: greedy and small-k rows that fit in registers take the streaming path
  int32_t xcap;            // extras capacity in LDS (unique history + tail)
  float* xl_glob;          // per-row extras in the workspace for longer histories (2 * xg_cap words a row), or NULL
  int32_t xg_cap;          // their capacity (unique history + tail)
  uint32_t off_bm, off_xl, off_cand, off_hist;   // LDS byte offsets
};

struct Misc {
  BlockScratch red;
  int32_t xl_n;
  int32_t cand_n;
  int32_t flags;
  int32_t ib[13];
  float fb[8];
  double db[8];
};

// ------------------------------------------------------------ element traits
struct F32 {
  static constexpr int EPC = 4;
  static constexpr int SZ = 4;
  __device__ static __forceinline__ float elem(const uint4& c, int e) {
    uint32_t d = e == 0 ? c.x : e == 1 ? c.y : e == 2 ? c.z : c.w;
    return __uint_as_float(d);
  }
  __device__ static __forceinline__ float load1(const unsigned char* row, int64_t i) {
    return ((const float*)row)[i];
  }
  __device__ static __forceinline__ uint32_t bits(const uint32_t* bm, int64_t c) {
    return (bm[c >> 3] >> ((uint32_t)(c & 7) * 4u)) & 0xfu;
  }
  __device__ static __forceinline__ uint4 mask(uint4 c, uint32_t b) {
    const uint32_t NI = 0xff800000u;
    c.x = (b & 1u) ? NI : c.x;
    c.y = (b & 2u) ? NI : c.y;
    c.z = (b & 4u) ? NI : c.z;
    c.w = (b & 8u) ? NI : c.w;
    return c;
  }
};
struct BF16 {
  static constexpr int EPC = 8;
  static constexpr int SZ = 2;
  __device__ static __forceinline__ float elem(const uint4& c, int e) {
    uint32_t d = (e >> 1) == 0 ? c.x : (e >> 1) == 1 ? c.y : (e >> 1) == 2 ? c.z : c.w;
    return __uint_as_float((e & 1) ? (d & 0xffff0000u) : (d << 16));
  }
  __device__ static __forceinline__ float load1(const unsigned char* row, int64_t i) {
    return __uint_as_float((uint32_t)((const uint16_t*)row)[i] << 16);
  }
  __device__ static __forceinline__ uint32_t bits(const uint32_t* bm, int64_t c) {
    return (bm[c >> 2] >> ((uint32_t)(c & 3) * 8u)) & 0xffu;
  }
  __device__ static __forceinline__ uint32_t mk(uint32_t b2) {
    return ((b2 & 1u) ? 0x0000ffffu : 0u) | ((b2 & 2u) ? 0xffff0000u : 0u);
  }
  __device__ static __forceinline__ uint4 mask(uint4 c, uint32_t b) {
    const uint32_t NI = 0xff80ff80u;
    uint32_t m;
    m = mk(b); c.x = (c.x & ~m) | (NI & m);
    m = mk(b >> 2); c.y = (c.y & ~m) | (NI & m);
    m = mk(b >> 4); c.z = (c.z & ~m) | (NI & m);
    m = mk(b >> 6); c.w = (c.w & ~m) | (NI & m);
    return c;
  }
};

template <typename T>
__device__ __forceinline__ float chunk_max(const uint4& c) {
  float m = T::elem(c, 0);
#pragma unroll
  for (int e = 1; e < T::EPC; ++e) m = fmax_nan(m, T::elem(c, e));
  return m;
}

__device__ __forceinline__ float penalize(float x, float pen, float rpen, bool recip) {
  // sampler.py:37: torch.where(score < 0, score * p, score / p), float32; recip: the positive
  // branch as x * rpen, rpen = RN(1/p), as torch computes it on a GPU
  return x < 0.0f ? x * pen : (recip ? x * rpen : x / pen);
}

// Smallest x with RN(x / tdiv) == RN(tau / tdiv): every x whose scaled value
// ties the scaled tau.  Searches the float order downwards from tau.
__device__ __forceinline__ float lower_preimage(float tau, float tdiv, float rdiv) {
  if (tdiv == 1.0f || !(__builtin_fabsf(tau) <= 3.4028235e38f)) return tau;
  const float ft = div_rn(tau, tdiv, rdiv);
  uint32_t khi = fkey(tau);
  uint32_t w = 16u + 4u * (uint32_t)__builtin_fminf(__builtin_ceilf(tdiv), 8.0e6f);
  uint32_t klo = khi > w ? khi - w : 0u;
  if (div_rn(fkey_inv(klo), tdiv, rdiv) >= ft) {
    klo = khi > (1u << 25) ? khi - (1u << 25) : 0u;
    if (div_rn(fkey_inv(klo), tdiv, rdiv) >= ft) return fkey_inv(klo);
  }
  while (klo + 1u < khi) {
    uint32_t mid = klo + (khi - klo) / 2u;
    if (div_rn(fkey_inv(mid), tdiv, rdiv) >= ft) khi = mid; else klo = mid;
  }
  return fkey_inv(khi);
}

// lower_preimage by a whole wave (every lane active, the same arguments in every lane): when
// the search window [khi - w, khi] fits the wave's 64 lanes, every key of it is tested at once,
// one per lane, and the first key that maps to RN(tau / t) or above is the answer (the mapping
// is monotone in the key); otherwise, and when the window's first key already maps there (the
// serial search then widens the window), the serial search.
__device__ __forceinline__ float wave_lower_preimage(float tau, float tdiv, float rdiv) {
  if (tdiv == 1.0f || !(__builtin_fabsf(tau) <= 3.4028235e38f)) return tau;
  const uint32_t khi = fkey(tau);
  const uint32_t w = 16u + 4u * (uint32_t)__builtin_fminf(__builtin_ceilf(tdiv), 8.0e6f);
  if (w > 63u || khi < w) return lower_preimage(tau, tdiv, rdiv);
  const float ft = div_rn(tau, tdiv, rdiv);
  const uint32_t l = (uint32_t)lane_id();
  const uint64_t m = ballot(l <= w && div_rn(fkey_inv(khi - w + (l <= w ? l : 0u)), tdiv, rdiv) >= ft);
  if (m & 1ull) return lower_preimage(tau, tdiv, rdiv);
  return fkey_inv(khi - w + (uint32_t)__builtin_ctzll(m));
}

// --------------------------------------------------------------- LDS sorts
// Ascending bitonic sort of P (power of two, 2..CAP) u64 keys in LDS.
__device__ __forceinline__ void lds_bitonic_sort(uint64_t* s, int P) {
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < (P >> 1); i += NT) {
        int lo = 2 * i - (i & (stride - 1));
        int hi = lo + stride;
        bool up = (lo & size) == 0;
        uint64_t a = s[lo], b = s[hi];
        if ((a > b) == up) { s[lo] = b; s[hi] = a; }
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ int next_pow2(int n) {
  int p = 2;
  while (p < n) p <<= 1;
  return p;
}

// Fixed-point mass: e in [0, 1] scaled by 2^40 (deterministic integer sums).
__device__ __forceinline__ uint64_t mass_fx(float e) {
  return (uint64_t)((double)e * 1099511627776.0);
}
constexpr double FX_INV = 1.0 / 1099511627776.0;

}  // namespace ns
