// gfx950 segment kernel: the sampler's fast path for greedy rows and top-k rows
// with k <= KFAST (sampler.py:31-89 for those rows).
//
// Each sampled row is cut into S segments of SEG_CH 16-byte chunks; one
// 256-thread workgroup per (row, segment), SCPT chunks per thread, all loads of
// a thread issued together (one HBM round trip per workgroup; at the decode
// batch every workgroup is resident at once).  Workgroups of one row are mapped
// to the same XCD (the dispatcher deals workgroup ids to the 8 XCDs
// round-robin), so a row's history ids and candidates stay in one L2.
//
// Per segment, per element only a NaN-propagating chunk maximum is computed:
//   * repetition penalty (sampler.py:34-38): the row's history ids falling in
//     the segment set bits of an LDS bitmap; each id that sets its bit first
//     (set semantics) is gathered, penalized and kept as an "extra" element.
//     History positions are skipped in the chunk data wherever exact values
//     matter (candidates, greedy), and chunks holding one are not used as
//     threshold sources.
//   * greedy rows: masked segment max and first index of the max (sampler.py:82-83).
//   * top-k rows: a lower bound tau of the row's k-th largest scaled logit from
//     the thread maxima (the ceil(k/4)-th largest of each wave's 64 thread
//     maxima, minimum over the 4 waves: at least k distinct elements reach it);
//     chunks whose maximum reaches tau are re-read (L2) and their elements >= tau
//     written as candidates (scaled value, token id).
// The last workgroup of a row to finish (atomic arrival counter) finalises the
// row: NaN/inf guard, the candidates above the largest segment bound, a
// histogram refinement, then exact top-k (ties kept), top-p, softmax and the
// inverse-CDF draw inside one wave over at most 256 survivors.  Rows it cannot
// resolve there (candidate overflow, huge tie groups) are flagged in `status`
// and resolved by the one-workgroup-per-row kernel launched after this one.
#pragma once

#include "ns_sample_kernel.h"

namespace ns {

constexpr int SNT = 256;               // threads per segment workgroup
constexpr int SNW = SNT / 64;          // waves per segment workgroup
constexpr int SCPT = 16;               // 16-byte chunks per thread
constexpr int SEG_CH = SNT * SCPT;     // chunks per segment
constexpr int SEG_CAP = 1024;          // candidate slots per segment (workspace)
constexpr int KFAST = 64;              // largest top_k resolved by the segment path
constexpr int XCAP = 2048;             // unique history ids per segment kept as extras
constexpr int FIN_SLOTS = 8;           // candidates per finaliser thread (FIN_SLOTS * SNT gathered)
constexpr int WAVE_CAP = 256;          // survivors finalised inside one wave
constexpr int SHIST = 256;             // refinement histogram bins
constexpr int HBATCH = 8;              // history ids per thread per batch
constexpr int MAX_SEGS = 16;           // segments per row (vocab <= 262144 at 16384 fp32 per segment)

constexpr int PATH_WAVE_SET = 6;       // out_info path code: top-k set finalised inside one wave
constexpr int SFLAG_NAN = 1 << 16;     // segment statistics: a NaN among the penalized values
constexpr int SFLAG_PINF = 1 << 17;    // segment statistics: a +inf among the penalized values
constexpr int SFLAG_XOVER = 1 << 18;   // segment statistics: more than XCAP unique history ids

struct SegStat {
  float ymax;       // segment max of the scaled logits (NaN-propagating)
  int32_t amax;     // greedy rows: first token id of the max
  float tau;        // top-k rows: lower bound of the row's k-th largest scaled logit
  int32_t ncand;    // candidates >= tau found (may exceed SEG_CAP: overflow)
  int32_t flags;    // FLAG_* row flags | SFLAG_* segment flags
  int32_t pad[3];
};

struct SegParams {
  const void* logits;
  int64_t row_stride;
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
  int32_t n_sample;
  int32_t S;             // segments per row
  int32_t* counters;     // [rows] arrival counters, zero between calls
  int32_t* status;       // [rows] written for every row: 1 = resolve in the per-row kernel
  SegStat* stats;        // [rows * S]
  uint64_t* cand;        // [rows * S * SEG_CAP]  (float bits << 32) | token id
};

// Rows this path resolves: greedy, or top-k with 1 <= k <= KFAST (and k < V, sampler.py:55).
__host__ __device__ __forceinline__ bool seg_row(float t, int32_t k, int64_t V) {
  return t == 0.0f || (k >= 1 && k <= KFAST && (int64_t)k < V);
}

// ------------------------------------------------------------ register access
// Raw float of element j (0 <= j < SCPT * EPC) of the thread's chunks, by selects
// (no dynamically indexed register arrays).
template <typename T>
__device__ __forceinline__ float elem_dyn(const uint4 (&v)[SCPT], int j) {
  const int dw = (j * T::SZ) >> 2;   // dword 0 .. 4*SCPT-1
  const int q = dw >> 2, c = dw & 3;
  uint32_t x = v[0].x, y = v[0].y, z = v[0].z, w = v[0].w;
#pragma unroll
  for (int i = 1; i < SCPT; ++i) {
    const bool s = q == i;
    x = s ? v[i].x : x;
    y = s ? v[i].y : y;
    z = s ? v[i].z : z;
    w = s ? v[i].w : w;
  }
  uint32_t d = x;
  d = c == 1 ? y : d;
  d = c == 2 ? z : d;
  d = c == 3 ? w : d;
  if (T::EPC == 8) return __uint_as_float((j & 1) ? (d & 0xffff0000u) : (d << 16));
  return __uint_as_float(d);
}

template <typename T>
__device__ __forceinline__ uint4 seg_ninf() {
  const uint32_t w = T::EPC == 8 ? 0xff80ff80u : 0xff800000u;
  return make_uint4(w, w, w, w);
}

// Chunk c of a row that ends past V: elements at or beyond V read as -inf
// (never loaded); the others are loaded one by one.
template <typename T>
__device__ __forceinline__ uint4 load_tail_chunk(const unsigned char* rowp, int64_t c, int64_t V) {
  const int64_t e0 = c * T::EPC;
  uint4 r = seg_ninf<T>();
  if (e0 < V) {
    uint32_t d[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < T::EPC; ++e) {
      if (e0 + e < V) {
        const uint32_t bits = __float_as_uint(T::load1(rowp, e0 + e));
        if (T::EPC == 8) {
          const int di = e >> 1;
          d[di] = (e & 1) ? ((d[di] & 0x0000ffffu) | (bits & 0xffff0000u)) : ((d[di] & 0xffff0000u) | (bits >> 16));
        } else {
          d[e] = bits;
        }
      }
    }
    r = make_uint4(d[0], d[1], d[2], d[3]);
  }
  return r;
}

// ------------------------------------------------- cross-workgroup exchange
// Candidates and segment statistics pass between workgroups of one launch
// through device-coherent accesses (relaxed agent-scope atomic loads/stores:
// they bypass the per-XCD L2's non-coherent state), so the arrival protocol
// needs no cache-wide write-back or invalidation.
__device__ __forceinline__ void dc_store(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t dc_load(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void dc_store_stat(SegStat* p, const SegStat& s) {
  const uint64_t* w = reinterpret_cast<const uint64_t*>(&s);
  uint64_t* d = reinterpret_cast<uint64_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) dc_store(d + i, w[i]);
}
__device__ __forceinline__ SegStat dc_load_stat(const SegStat* p) {
  SegStat s;
  uint64_t* w = reinterpret_cast<uint64_t*>(&s);
  const uint64_t* d = reinterpret_cast<const uint64_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = dc_load(d + i);
  return s;
}

// ------------------------------------------------------------ wave sorting

// Ascending bitonic sort of 64*R keys held by one wave: element i = r*64 + lane.
template <int R>
__device__ __forceinline__ void wave_sort_u64(uint64_t (&a)[R]) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= 64 * R; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= 64) {
        const int rs = stride >> 6;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if ((r & rs) == 0) {
            const int i = r * 64 + lane;
            const bool up = (i & size) == 0;
            const uint64_t x = a[r], y = a[r | rs];
            const uint64_t mn = x < y ? x : y, mx = x < y ? y : x;
            a[r] = up ? mn : mx;
            a[r | rs] = up ? mx : mn;
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint64_t p = lane_xor(a[r], stride);
          const int i = r * 64 + lane;
          const bool up = (i & size) == 0;
          const bool lower = (lane & stride) == 0;
          const bool keep_min = lower == up;
          const uint64_t mn = a[r] < p ? a[r] : p, mx = a[r] < p ? p : a[r];
          a[r] = keep_min ? mn : mx;
        }
      }
    }
  }
}

// Ascending bitonic sort of 64 u32 keys (one per lane).
__device__ __forceinline__ uint32_t wave_sort_u32(uint32_t a) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint32_t p = lane_xor(a, stride);
      const bool up = (lane & size) == 0;
      const bool lower = (lane & stride) == 0;
      a = (lower == up) ? (a < p ? a : p) : (a < p ? p : a);
    }
  }
  return a;
}

// Ascending bitonic sort of 64*R u32 keys held by one wave: element i = r*64 + lane.
template <int R>
__device__ __forceinline__ void wave_sort_u32r(uint32_t (&a)[R]) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= 64 * R; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= 64) {
        const int rs = stride >> 6;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if ((r & rs) == 0) {
            const bool up = ((r * 64 + lane) & size) == 0;
            const uint32_t x = a[r], y = a[r | rs];
            const uint32_t mn = x < y ? x : y, mx = x < y ? y : x;
            a[r] = up ? mn : mx;
            a[r | rs] = up ? mx : mn;
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint32_t p = lane_xor(a[r], stride);
          const bool up = ((r * 64 + lane) & size) == 0;
          const bool lower = (lane & stride) == 0;
          a[r] = (lower == up) ? (a[r] < p ? a[r] : p) : (a[r] < p ? p : a[r]);
        }
      }
    }
  }
}

// Inclusive prefix sums of 64*R doubles in element order i = r*64 + lane.
template <int R>
__device__ __forceinline__ void wave_scan_rows(const double (&v)[R], double (&out)[R]) {
  double carry = 0.0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const double s = wave_incl_scan(v[r]);
    out[r] = carry + s;
    carry += read_lane(s, 63);
  }
}

// Shared memory of the segment workgroup.
struct SegSmem {
  uint32_t bm[SEG_CH * 8 / 32];     // history bitmap of the segment (8 elements per chunk max)
  int32_t xl_id[XCAP];              // unique history ids of the segment
  float xl_val[XCAP];               // their penalized values
  uint64_t list[WAVE_CAP];          // finaliser survivors
  uint32_t hist[SHIST];             // finaliser refinement histogram
  int32_t off[MAX_SEGS + 1];        // finaliser candidate offsets per segment
  float fred[SNW];
  int32_t ired[SNW];
  int32_t wbase[SNW];
  int32_t cnt;
  int32_t last;
  int32_t flags;
  float fb[4];
  int32_t ib[8];
};

// Block reductions over the 4 waves (two barriers each).
__device__ __forceinline__ float seg_max_nan(float v, SegSmem* sm) {
  v = wave_max_nan(v);
  if (lane_id() == 0) sm->fred[wave_id()] = v;
  __syncthreads();
  float r = sm->fred[0];
#pragma unroll
  for (int w = 1; w < SNW; ++w) r = fmax_nan(r, sm->fred[w]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ float seg_min_f(float v, SegSmem* sm) {
  v = wave_min(v);
  if (lane_id() == 0) sm->fred[wave_id()] = v;
  __syncthreads();
  float r = sm->fred[0];
#pragma unroll
  for (int w = 1; w < SNW; ++w) r = sm->fred[w] < r ? sm->fred[w] : r;
  __syncthreads();
  return r;
}
__device__ __forceinline__ int32_t seg_min_i(int32_t v, SegSmem* sm) {
  v = wave_min(v);
  if (lane_id() == 0) sm->ired[wave_id()] = v;
  __syncthreads();
  int32_t r = sm->ired[0];
#pragma unroll
  for (int w = 1; w < SNW; ++w) r = sm->ired[w] < r ? sm->ired[w] : r;
  __syncthreads();
  return r;
}
// Exclusive prefix sum over the 4 waves' threads; *total receives the sum (two barriers).
__device__ __forceinline__ int32_t seg_excl_i(int32_t v, int32_t* total, SegSmem* sm) {
  const int32_t inc = wave_incl_scan(v);
  if (lane_id() == 63) sm->ired[wave_id()] = inc;
  __syncthreads();
  int32_t off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < SNW; ++w) {
    const int32_t t = sm->ired[w];
    if (w < wave_id()) off += t;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return off + inc - v;
}
__device__ __forceinline__ int32_t seg_sum_i(int32_t v, SegSmem* sm) {
  v = wave_sum(v);
  if (lane_id() == 0) sm->ired[wave_id()] = v;
  __syncthreads();
  int32_t r = 0;
#pragma unroll
  for (int w = 0; w < SNW; ++w) r += sm->ired[w];
  __syncthreads();
  return r;
}

__device__ __forceinline__ void seg_write_info(int32_t* out_info, int row, int32_t path, int32_t n_kept, float thr,
                                               int32_t n_topk, int32_t n_cand, int32_t flags, float vstar,
                                               int32_t istar) {
  if (out_info == nullptr) return;
  int32_t* w = out_info + (int64_t)row * INFO_WORDS;
  w[0] = path; w[1] = n_kept; w[2] = (int32_t)__float_as_uint(thr); w[3] = n_topk;
  w[4] = n_cand; w[5] = flags; w[6] = (int32_t)__float_as_uint(vstar); w[7] = istar;
}

// Element i = r*64 + l of a wave's register rows, r and l wave-uniform, read through
// scalar registers (a select over a[r] would become a dynamically indexed array).
template <int R>
__device__ __forceinline__ uint64_t wave_elem(const uint64_t (&a)[R], int i) {
  const int rr = i >> 6, l = i & 63;
  uint64_t x = read_lane(a[0], l);
#pragma unroll
  for (int r = 1; r < R; ++r) {
    const uint64_t t = read_lane(a[r], l);
    x = r == rr ? t : x;
  }
  return x;
}

// Top-p, softmax and inverse-CDF draw by one wave over the nk survivors of the
// top-k cut, given in a[] (element i = r*64 + lane) in sorted order: scaled value
// descending, token id ascending.  M is the row maximum and thr the k-th largest
// value (-inf when fewer than k candidates); entries at i >= nk are ignored.
template <int R>
__device__ __forceinline__ void wave_select_draw(const uint64_t (&a)[R], int nk, float M, float thr, bool topp_on,
                                                 float p32, float u, int row, const IdSink& out_ids, float* out_probs,
                                                 int64_t V, int32_t* out_info, int32_t flags, int32_t n_cand,
                                                 int32_t path) {
  const int lane = lane_id();
  // softmax numerators over the kept prefix (sampler.py:65 / :76)
  float ev[R];
  double es[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * 64 + lane;
    ev[r] = i < nk ? ns_expf(desc_key_val(a[r]) - M) : 0.0f;
    es[r] = (double)ev[r];
  }
  int nf = nk;
  float vstar = -__builtin_inff();
  int32_t istar = -1;
  if (topp_on) {
    double z = 0.0;
#pragma unroll
    for (int r = 0; r < R; ++r) z += wave_sum(es[r]);
    double qv[R], cs[R];
#pragma unroll
    for (int r = 0; r < R; ++r) qv[r] = (double)(float)(es[r] / z);
    wave_scan_rows<R>(qv, cs);
    // first sorted position whose float32 prefix exceeds top_p; it is kept (sampler.py:66-72)
    int J = -1;
#pragma unroll
    for (int r = R - 1; r >= 0; --r) {
      const int i = r * 64 + lane;
      const uint64_t m = ballot(i < nk && (float)cs[r] > p32);
      if (m != 0ull) J = r * 64 + __builtin_ctzll(m);
    }
    if (J >= 0) nf = J + 1;
    const uint64_t kc = wave_elem<R>(a, nf - 1);
    vstar = desc_key_val(kc);
    istar = (int32_t)desc_key_id(kc);
  }
  // final probabilities over the nf kept tokens, then the draw in token-id order
  double z2 = 0.0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * 64 + lane;
    z2 += wave_sum(i < nf ? es[r] : 0.0);
  }
  // ids[r] / ps[r]: the kept tokens and their probabilities in ascending id order
  uint32_t ids[R];
  float ps[R];
  if constexpr (R == 1) {
    // one register row: sort (id << 6 | lane) as 32-bit keys (ids < 2^18), then fetch
    // each probability from the lane it came from
    const float pv = lane < nf ? (float)(es[0] / z2) : 0.0f;
    uint32_t key = lane < nf ? ((desc_key_id(a[0]) << 6) | (uint32_t)lane) : 0xffffffffu;
    key = wave_sort_u32(key);
    ps[0] = __int_as_float(__builtin_amdgcn_ds_bpermute((int)((key & 63u) << 2), __float_as_int(pv)));
    ids[0] = key >> 6;
  } else {
    uint64_t b[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = r * 64 + lane;
      b[r] = ~0ull;
      if (i < nf) {
        const float pv = (float)(es[r] / z2);
        b[r] = ((uint64_t)desc_key_id(a[r]) << 32) | __float_as_uint(pv);
      }
    }
    wave_sort_u64<R>(b);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      ids[r] = (uint32_t)(b[r] >> 32);
      ps[r] = __uint_as_float((uint32_t)b[r]);
    }
  }
  double pd[R], cd[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * 64 + lane;
    pd[r] = i < nf ? (double)ps[r] : 0.0;
  }
  wave_scan_rows<R>(pd, cd);
  const double ud = (double)u;
  int pick = -1, lastpos = -1;
#pragma unroll
  for (int r = R - 1; r >= 0; --r) {
    const int i = r * 64 + lane;
    const uint64_t m = ballot(i < nf && cd[r] > ud);
    if (m != 0ull) pick = r * 64 + __builtin_ctzll(m);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * 64 + lane;
    const uint64_t m = ballot(i < nf && pd[r] > 0.0);
    if (m != 0ull) lastpos = r * 64 + 63 - __builtin_clzll(m);
  }
  int32_t fl = flags;
  if (pick < 0) { pick = lastpos >= 0 ? lastpos : 0; fl |= FLAG_LOCATE_FALLBACK; }
  {
    uint32_t idp = read_lane(ids[0], pick & 63);
#pragma unroll
    for (int r = 1; r < R; ++r) {
      const uint32_t t = read_lane(ids[r], pick & 63);
      idp = (pick >> 6) == r ? t : idp;
    }
    if (lane == 0) {
      put_id(out_ids, row, (int64_t)idp);
      seg_write_info(out_info, row, path, nf, thr, nk, n_cand, fl, vstar, istar);
    }
  }
  if (out_probs != nullptr) {
    float* pr = out_probs + (int64_t)row * V;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = r * 64 + lane;
      if (i < nf) pr[ids[r]] = ps[r];
    }
  }
}

// Exact top-k (ties kept), top-p, softmax and inverse-CDF draw over n <= 64*R
// survivors, run by one wave.  list[i] = (float bits << 32) | token id where the
// float is a logit after the penalty; it is scaled here by the row's temperature
// (tdiv, rdiv = RN(1/tdiv)); pass tdiv = rdiv = 1 for values already scaled.
// Every survivor is >= the row's k-th largest scaled value and the row maximum
// is among them.
template <int R>
__device__ __forceinline__ void wave_finalize(const uint64_t* list, int n, int k, bool topp_on, float p32, float tdiv, float rdiv,
                              float u, int row, const IdSink& out_ids, float* out_probs, int64_t V, int32_t* out_info,
                              int32_t flags, int32_t n_cand, int32_t path) {
  const int lane = lane_id();
  uint64_t a[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * 64 + lane;
    a[r] = ~0ull;
    if (i < n) {
      const uint64_t e = list[i];
      a[r] = desc_key(div_rn(__uint_as_float((uint32_t)(e >> 32)), tdiv, rdiv), (uint32_t)e);
    }
  }
  wave_sort_u64<R>(a);   // value descending, token id ascending
  const float M = desc_key_val(read_lane(a[0], 0));   // the row maximum

  // top-k threshold: the k-th largest (sampler.py:56-58); every value >= it is kept
  float thr = -__builtin_inff();
  if (n >= k) {
    thr = desc_key_val(wave_elem<R>(a, k - 1));
  }
  int nk = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * 64 + lane;
    nk += __popcll(ballot(i < n && desc_key_val(a[r]) >= thr));
  }
  wave_select_draw<R>(a, nk, M, thr, topp_on, p32, u, row, out_ids, out_probs, V, out_info, flags, n_cand, path);
}

// Tail of the workgroup finaliser: wave 0 loads the first nk sorted keys from LDS.
template <int R>
__device__ __forceinline__ void wave_select_draw_lds(const uint64_t* sorted, int nk, float M, float thr, bool topp_on, float p32,
                                     float u, int row, const IdSink& out_ids, float* out_probs, int64_t V,
                                     int32_t* out_info, int32_t flags, int32_t n_cand, int32_t path) {
  const int lane = lane_id();
  uint64_t a[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * 64 + lane;
    a[r] = i < nk ? sorted[i] : ~0ull;
  }
  wave_select_draw<R>(a, nk, M, thr, topp_on, p32, u, row, out_ids, out_probs, V, out_info, flags, n_cand, path);
}

// Top-p, softmax and inverse-CDF draw by one wave over the nk <= 64 survivors of the
// top-k cut, the ordering already done by the workgroup: a holds the sorted keys
// (element i = lane; scaled value descending, token id ascending), byid[0..n) the same
// n <= 128 candidates in ascending token-id order and vr[0..n) the sorted position of
// each.  One float64 prefix sum of the softmax numerators gives both normalisers (the
// top-k set's and the kept set's, sampler.py:65 and :76), and the draw runs over the
// id-ordered candidates with probability 0 for those not kept, so nothing is sorted
// here.  Probabilities are the float32 roundings of the numerators times the float64
// reciprocal of the normaliser.
__device__ __forceinline__ void wave_draw_sorted(uint64_t a, int nk, int n, const uint64_t* byid, const int32_t* vr,
                                                 float M, float thr, bool topp_on, float p32, float u, int row,
                                                 const IdSink& out_ids, float* out_probs, int64_t V, int32_t* out_info,
                                                 int32_t flags, int32_t n_cand, int32_t path) {
  const int lane = lane_id();
  const uint64_t b0 = lane < n ? byid[lane] : ~0ull;
  const uint64_t b1 = 64 + lane < n ? byid[64 + lane] : ~0ull;
  const int r0 = lane < n ? vr[lane] : 64;
  const int r1 = 64 + lane < n ? vr[64 + lane] : 64;
  const float ev = lane < nk ? ns_expf(desc_key_val(a) - M) : 0.0f;
  // the numerators in id order, ahead of the cut they do not depend on
  const float e0 = ns_expf(desc_key_val(b0) - M), e1 = ns_expf(desc_key_val(b1) - M);
  const double cs = wave_incl_scan((double)ev);
  int nf = nk;
  float vstar = -__builtin_inff();
  int32_t istar = -1;
  if (topp_on) {
    // first sorted position whose float32 prefix exceeds top_p; it is kept (sampler.py:66-72).
    // The prefix of the top-k softmax is taken as the float64 prefix of the numerators times
    // the reciprocal of their sum: it differs from the sum of float32-rounded probabilities
    // by about 1e-7, inside the 1e-6 zone where the cut is ambiguous anyway.
    const double rz = rcp_f64(read_lane(cs, nk - 1));
    const uint64_t m = ballot(lane < nk && (float)(cs * rz) > p32);
    if (m != 0ull) nf = __builtin_ctzll(m) + 1;
    const uint64_t kc = read_lane(a, nf - 1);
    vstar = desc_key_val(kc);
    istar = (int32_t)desc_key_id(kc);
  }
  const double rz2 = rcp_f64(read_lane(cs, nf - 1));
  // final probabilities of the kept candidates (sorted position < nf), in id order
  const bool k0 = r0 < nf, k1 = r1 < nf;
  const float p0 = k0 ? (float)((double)e0 * rz2) : 0.0f;
  const float p1 = k1 ? (float)((double)e1 * rz2) : 0.0f;
  const double c0 = wave_incl_scan((double)p0);
  const double c1 = read_lane(c0, 63) + wave_incl_scan((double)p1);
  // the first id-order position whose cumulative mass exceeds u (sampler.py:87 as an
  // inverse CDF); the mass only grows at kept positions
  const double ud = (double)u;
  const uint64_t m0 = ballot(c0 > ud), m1 = ballot(c1 > ud);
  int pick = m0 != 0ull ? __builtin_ctzll(m0) : (m1 != 0ull ? 64 + __builtin_ctzll(m1) : -1);
  int32_t fl = flags;
  if (pick < 0) {
    // rounding left the total at or below u: the last kept position with mass
    const uint64_t l0 = ballot(p0 > 0.0f), l1 = ballot(p1 > 0.0f);
    const uint64_t q0 = ballot(k0), q1 = ballot(k1);
    pick = l1 != 0ull ? 127 - __builtin_clzll(l1)
         : l0 != 0ull ? 63 - __builtin_clzll(l0)
         : q0 != 0ull ? __builtin_ctzll(q0) : 64 + __builtin_ctzll(q1);
    fl |= FLAG_LOCATE_FALLBACK;
  }
  const uint32_t i0 = read_lane(desc_key_id(b0), pick & 63), i1 = read_lane(desc_key_id(b1), pick & 63);
  if (lane == 0) {
    put_id(out_ids, row, (int64_t)(pick < 64 ? i0 : i1));
    seg_write_info(out_info, row, path, nf, thr, nk, n_cand, fl, vstar, istar);
  }
  if (out_probs != nullptr) {
    float* pr = out_probs + (int64_t)row * V;
    if (k0) pr[desc_key_id(b0)] = p0;
    if (k1) pr[desc_key_id(b1)] = p1;
  }
}

// Keys of slice s of the list (PER entries) below ki (c) and with a token id below ki's
// (ci).  Every read is issued before the first compare.
template <int PER>
__device__ __forceinline__ void rank_slice(const uint64_t* list, int s, uint64_t ki, int& c, int& ci) {
  const uint64_t* sl = list + s * PER;
  uint64_t a[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) a[j] = sl[j];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    c += a[j] < ki ? 1 : 0;
    ci += (uint32_t)a[j] < (uint32_t)ki ? 1 : 0;
  }
}

// The same selection and draw as wave_finalize over n <= WAVE_CAP survivors, with the
// ordering done by the whole workgroup (NTH threads, all of which must call it).
// Entry: list[0..n) holds the sort keys (desc_key of the scaled value and token id),
// list[n..WAVE_CAP) holds ~0 (it sorts after every key), and a workgroup barrier has
// passed since both were written; k <= 64.  out[] is a region apart from the list of
// 2 * WAVE_CAP entries: the keys land in order in out[0..n), and for n <= 128 also in
// ascending token-id order in out[WAVE_CAP..), with their sorted positions behind them.
// A key's position is the number of keys below it: G consecutive lanes take one key,
// each counts one slice of the list, and the group's counts are summed by lane
// exchanges (no atomics, no second barrier).  Wave 0 then runs top-p, softmax and the
// draw over the top-k prefix.
// The ordering step alone: out[0..n) the keys in order, and for n <= WAVE_CAP / 2 also
// out[WAVE_CAP..) in ascending token-id order with their sorted positions behind them.
// Same entry conditions as block_finalize_keys; the caller places the barrier after it.
template <int NTH>
__device__ __forceinline__ void block_rank_keys(const uint64_t* list, uint64_t* out, int n) {
  static_assert(NTH == 4 * WAVE_CAP, "8 lanes per key up to WAVE_CAP / 2 keys, 4 lanes per key beyond");
  const int tid = threadIdx.x;
  uint64_t* sorted = out;
  uint64_t* byid = out + WAVE_CAP;
  int32_t* vr = reinterpret_cast<int32_t*>(out + WAVE_CAP + WAVE_CAP / 2);
  const bool g8 = n <= WAVE_CAP / 2;
  {
    const int G = g8 ? 8 : 4;
    const int i = g8 ? tid >> 3 : tid >> 2;
    const int s = tid & (G - 1);
    const uint64_t ki = list[i];
    int c = 0, ci = 0;
    if (g8) {
      // slice s: [s * PER, s * PER + PER), PER = ceil(n / 8) rounded up to 2 mod 4 (<= 18),
      // so the 8 slices start in distinct LDS banks; the padding past n never counts and
      // waves whose keys all lie past n skip the count.  ci counts the smaller token ids.
      if (wave_id() * 8 < n) {
        const int cls = (((n + 7) >> 3) + 1) >> 2;   // PER = 4 * cls + 2
        if (cls == 0) rank_slice<2>(list, s, ki, c, ci);
        else if (cls == 1) rank_slice<6>(list, s, ki, c, ci);
        else if (cls == 2) rank_slice<10>(list, s, ki, c, ci);
        else if (cls == 3) rank_slice<14>(list, s, ki, c, ci);
        else rank_slice<18>(list, s, ki, c, ci);
      }
    } else {
      const uint64_t* sl = list + s * (WAVE_CAP / 4);
#pragma unroll 8
      for (int j = 0; j < WAVE_CAP / 4; ++j) c += sl[j] < ki ? 1 : 0;
    }
    c += lane_xor(c, 1);
    c += lane_xor(c, 2);
    if (g8) {
      c += lane_xor(c, 4);
      ci += lane_xor(ci, 1);
      ci += lane_xor(ci, 2);
      ci += lane_xor(ci, 4);
    }
    if (s == 0 && i < n) {
      sorted[c] = ki;
      if (g8) { byid[ci] = ki; vr[ci] = c; }
    }
  }
}

template <int NTH>
__device__ __forceinline__ void block_finalize_keys(const uint64_t* list, uint64_t* out, int n, int k, bool topp_on,
                                                    float p32, float u, int row, const IdSink& out_ids, float* out_probs,
                                                    int64_t V, int32_t* out_info, int32_t flags, int32_t n_cand,
                                                    int32_t path) {
  NS_STAMP_DECL;
  const int tid = threadIdx.x;
  uint64_t* sorted = out;
  uint64_t* byid = out + WAVE_CAP;
  int32_t* vr = reinterpret_cast<int32_t*>(out + WAVE_CAP + WAVE_CAP / 2);
  const bool g8 = n <= WAVE_CAP / 2;
  block_rank_keys<NTH>(list, out, n);
  __syncthreads();
  NS_STAMP(5);
  if (tid >= 64) return;
  // the first 128 sorted keys in registers: row maximum, k-th largest, kept count
  uint64_t a2[2];
  a2[0] = tid < n ? sorted[tid] : ~0ull;
  a2[1] = 64 + tid < n ? sorted[64 + tid] : ~0ull;
  const float M = desc_key_val(read_lane(a2[0], 0));   // the row maximum
  // top-k threshold: the k-th largest (sampler.py:56-58); every value >= it is kept
  const float thr = n >= k ? desc_key_val(read_lane(a2[0], k - 1)) : -__builtin_inff();
  int nk = __popcll(ballot(tid < n && desc_key_val(a2[0]) >= thr)) +
           __popcll(ballot(64 + tid < n && desc_key_val(a2[1]) >= thr));
  for (int base = 128; base < n && nk == base; base += 64) {   // tie group beyond 128 (rare)
    const int i = base + tid;
    nk += __popcll(ballot(i < n && desc_key_val(sorted[i < n ? i : 0]) >= thr));
  }
  NS_STAMP(10);   // wave 0: the top-k cut
  if (nk <= 64 && g8) {
    wave_draw_sorted(a2[0], nk, n, byid, vr, M, thr, topp_on, p32, u, row, out_ids, out_probs, V, out_info, flags,
                     n_cand, path);
  } else if (nk <= 64) {
    const uint64_t a1[1] = {a2[0]};
    wave_select_draw<1>(a1, nk, M, thr, topp_on, p32, u, row, out_ids, out_probs, V, out_info, flags, n_cand, path);
  } else if (nk <= 128) {
    wave_select_draw<2>(a2, nk, M, thr, topp_on, p32, u, row, out_ids, out_probs, V, out_info, flags, n_cand, path);
  } else {
    wave_select_draw_lds<4>(sorted, nk, M, thr, topp_on, p32, u, row, out_ids, out_probs, V, out_info, flags, n_cand,
                            path);
  }
}

// Wave-aggregated append of one candidate (scaled value y, token id) to the
// segment's workspace slots; callable from divergent code (active lanes only).
__device__ __forceinline__ void seg_append(float y, int64_t id, uint64_t* cbase, SegSmem* sm) {
  const uint64_t m = ballot(true);
  const int leader = __builtin_ctzll(m);
  int base = 0;
  if (lane_id() == leader) base = atomicAdd(&sm->cnt, __popcll(m));
  base = read_lane(base, leader);
  const int pos = base + lanes_below(m);
  if (pos < SEG_CAP) dc_store(cbase + pos, ((uint64_t)__float_as_uint(y) << 32) | (uint32_t)id);
}

// The segment kernel's work for this workgroup's (row, segment), with the workgroup's LDS.
template <typename T>
__device__ __forceinline__ void segment_body(const SegParams& P, SegSmem& sm) {
  constexpr int EPC = T::EPC;
  constexpr int SEG_EL = SEG_CH * EPC;         // elements per segment
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wid = wave_id();
  const int S = P.S;
  // XCD-aware mapping: all segments of a row share blockIdx % 8
  const int b = blockIdx.x;
  const int xcd = b & 7;
  const int i8 = b >> 3;
  const int rg = i8 / S;
  const int seg = i8 - rg * S;
  const int row = rg * 8 + xcd;
  if (row >= P.n_sample) return;
  const int64_t V = P.vocab;
  const float temp = P.temperature[row];
  const int32_t k = P.top_k[row];
  if (!seg_row(temp, k, V)) {                  // resolved by the per-row kernel
    if (seg == 0 && tid == 0) P.status[row] = 1;
    return;
  }
  const int64_t src = P.sample_idx ? P.sample_idx[row] : (int64_t)row;
  int32_t h0 = 0, h1 = 0;
  row_history(P.hist_off, P.hist_slot, P.hist_len, P.hist_nslots, P.hist_cap, row, h0, h1);
  if (src < 0 || src >= P.n_rows_total || h0 < 0 || h1 < h0 || h1 - h0 > MAX_HIST) {
    // invalid row: the per-row kernel reports it
    if (seg == 0 && tid == 0) P.status[row] = 1;
    return;
  }
  const unsigned char* rowp = (const unsigned char*)P.logits + src * P.row_stride * T::SZ;
  const uint4* rowv = reinterpret_cast<const uint4*>(rowp);
  const int64_t c0 = (int64_t)seg * SEG_CH;    // first chunk of the segment
  const int64_t e0 = c0 * EPC;                 // first element

  // ---- all row loads of this thread in flight at once
  uint4 v[SCPT];
  {
    // buffer loads over the row's full chunks: chunks past them read zero and are
    // replaced when first used
    const uint32_t nbytes = (uint32_t)((V / EPC) * 16);
#pragma unroll
    for (int q = 0; q < SCPT; ++q)
      v[q] = buf_load16_at(rowp, nbytes, (uint32_t)((c0 + q * SNT) * 16), (uint32_t)tid * 16u);
  }
  // chunks past the row's full chunks: -inf, and the chunk holding the last tokens
  // when V is not a multiple of EPC (its own register); replaced when first used
  const int64_t nfull_r = V / EPC;
  const bool has_tail = (nfull_r * EPC < V) && (nfull_r - c0) % SNT == tid && nfull_r >= c0 &&
                        nfull_r < c0 + SEG_CH;
  const uint4 vtail = has_tail ? load_tail_chunk<T>(rowp, nfull_r, V) : seg_ninf<T>();

  const float pen = P.penalty[row];
  const int32_t H = h1 - h0;
  const bool pen_on = pen != 1.0f && H > 0;    // sampler.py:33
  const bool greedy = temp == 0.0f;
  const float tdiv = temp > 0.0f ? __builtin_fmaxf(temp, 1e-6f) : 1.0f;   // sampler.py:42
  const float rdiv = 1.0f / tdiv;
  const bool recip = P.pen_rcp != nullptr;
  const float rpen = recip ? P.pen_rcp[row] : 1.0f / pen;
  auto pen_val = [&](float x) -> float { return pen_rn(x, pen, rpen, recip); };
  int32_t flags = 0;

  // ---- history: bitmap of the segment and the unique ids in it (set semantics)
  int U = 0;
  if (pen_on) {
    for (int i = tid; i < SEG_EL / 32; i += SNT) sm.bm[i] = 0u;
    if (tid == 0) sm.flags = 0;
    __syncthreads();
    const int32_t* hp = P.hist_ids + h0;
    bool bad = false;
    for (int base = 0; base < H; base += SNT * HBATCH) {
      int32_t hv[HBATCH];
#pragma unroll
      for (int s = 0; s < HBATCH; ++s) {
        const int j = base + s * SNT + tid;
        hv[s] = j < H ? hp[j] : 0;
      }
#pragma unroll
      for (int s = 0; s < HBATCH; ++s) {
        const int j = base + s * SNT + tid;
        if (j < H) {
          const int32_t id = hv[s];
          if (id < 0 || (int64_t)id >= V) {
            bad = true;
          } else if ((int64_t)id >= e0 && (int64_t)id < e0 + SEG_EL) {
            const int32_t l = id - (int32_t)e0;
            atomicOr(&sm.bm[l >> 5], 1u << (l & 31));
          }
        }
      }
    }
    if (bad) atomicOr(&sm.flags, FLAG_BAD_HIST_ID);
    __syncthreads();
    flags |= sm.flags;
    // the unique ids in ascending order, read off the finished bitmap (a list built by
    // appending in atomic order would hand the extras to threads in a different order
    // every run, and with them the segment's bound and candidate count)
    constexpr int WPT = SEG_EL / 32 / SNT;   // bitmap words per thread
    static_assert(WPT * SNT * 32 == SEG_EL, "segment bitmap split evenly over the threads");
    uint32_t wv[WPT];
    int32_t c = 0;
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
      wv[j] = sm.bm[tid * WPT + j];
      c += __popc(wv[j]);
    }
    int32_t pos = seg_excl_i(c, &U, &sm);
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
      uint32_t m = wv[j];
      while (m != 0u) {
        const int b = __builtin_ctz(m);
        m &= m - 1u;
        if (pos < XCAP) sm.xl_id[pos] = (int32_t)e0 + (tid * WPT + j) * 32 + b;
        ++pos;
      }
    }
    if (U > XCAP) { flags |= SFLAG_XOVER; U = XCAP; }
    __syncthreads();   // the list before the extras are gathered
  }

  // ---- extras: thread t gathers and penalizes entries t, t+SNT, ... (issued before the chunk work)
  constexpr int XPT = XCAP / SNT;
  float xr[XPT];
#pragma unroll
  for (int r = 0; r < XPT; ++r) {
    const int i = tid + r * SNT;
    xr[r] = i < U ? T::load1(rowp, sm.xl_id[i]) : 0.0f;
  }

  // ---- chunk maxima over the raw data; threshold sources skip chunks holding history positions
  float cm[SCPT];
  float tval = -__builtin_inff();             // max over distinct elements with exact (penalized) values
  bool nanf = false, pinf = false;            // NaN / +inf among the penalized values
  uint32_t hq = 0u;                           // bit q: chunk q holds a history position
#pragma unroll
  for (int q = 0; q < SCPT; ++q) {
    {
      const int64_t c = c0 + q * SNT + tid;
      if (c >= nfull_r) v[q] = c == nfull_r ? vtail : seg_ninf<T>();
    }
    cm[q] = chunk_max<T>(v[q]);
    const uint32_t hb = pen_on ? T::bits(sm.bm, q * SNT + tid) : 0u;
    hq |= (hb != 0u) ? (1u << q) : 0u;
    if (hb == 0u) tval = __builtin_fmaxf(tval, cm[q]);
    else if (greedy) cm[q] = chunk_max<T>(T::mask(v[q], hb));   // greedy rows: exact masked chunk max
    if (!(cm[q] <= 3.40282347e38f) && cm[q] != -__builtin_inff()) {   // NaN or +inf in the chunk (rare)
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        const float x = T::elem(v[q], e);
        if (!((hb >> e) & 1u)) { nanf |= x != x; pinf |= x == __builtin_inff(); }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < XPT; ++r) {
    const int i = tid + r * SNT;
    if (i < U) {
      const float pv = pen_val(xr[r]);
      sm.xl_val[i] = pv;
      xr[r] = pv;
      tval = __builtin_fmaxf(tval, pv);
      nanf |= pv != pv;
      pinf |= pv == __builtin_inff();
    }
  }
  if (ballot(nanf) != 0ull) flags |= SFLAG_NAN;
  if (ballot(pinf) != 0ull) flags |= SFLAG_PINF;
  if (lane == 0) sm.ired[wid] = flags;
  if (tid == 0) sm.cnt = 0;

  SegStat st;
  st.ncand = 0;
  st.tau = -__builtin_inff();
  st.amax = -1;
  st.ymax = -__builtin_inff();
  st.pad[0] = st.pad[1] = st.pad[2] = 0;
  uint64_t* cbase = P.cand + ((int64_t)row * S + seg) * SEG_CAP;

  if (greedy) {
    __syncthreads();
    // the waves' flags, read before the reductions below reuse their words
    const int32_t wfl = sm.ired[0] | sm.ired[1] | sm.ired[2] | sm.ired[3];
    // masked maximum and its first index (NaN counts as the max, sampler.py:82-83):
    // the masked chunk maxima, then an element scan (re-read from L2) of the first
    // chunk of each thread that reaches the segment maximum.
    float gm = -__builtin_inff();
#pragma unroll
    for (int q = 0; q < SCPT; ++q) gm = fmax_nan(gm, cm[q]);
#pragma unroll
    for (int r = 0; r < XPT; ++r)
      if (tid + r * SNT < U) gm = fmax_nan(gm, xr[r]);
    const float Mx = seg_max_nan(gm, &sm);
    const bool nanm = Mx != Mx;
    int32_t gi = 0x7fffffff;
#pragma unroll
    for (int q = 0; q < SCPT; ++q) {
      // chunks of a thread are in ascending token order: the first matching chunk decides
      if (gi == 0x7fffffff && (nanm ? (cm[q] != cm[q]) : (cm[q] == Mx))) {
        const uint32_t hb = pen_on ? T::bits(sm.bm, q * SNT + tid) : 0u;
        const int64_t c = c0 + q * SNT + tid;
        const uint4 raw = (c + 1) * EPC <= V ? rowv[c] : load_tail_chunk<T>(rowp, c, V);   // re-read (L2)
        const uint4 w = pen_on ? T::mask(raw, hb) : raw;
#pragma unroll
        for (int e = EPC - 1; e >= 0; --e) {
          const float x = T::elem(w, e);
          if ((nanm ? (x != x) : (x == Mx)) && c * EPC + e < V) gi = (int32_t)(c * EPC + e);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < XPT; ++r) {
      const int i = tid + r * SNT;
      if (i < U && (nanm ? (xr[r] != xr[r]) : (xr[r] == Mx)) && sm.xl_id[i] < gi) gi = sm.xl_id[i];
    }
    const int32_t best = seg_min_i(gi, &sm);
    st.ymax = Mx;
    st.amax = best;
    st.flags = flags | wfl;
  } else {
    // ---- lower bound of the k-th largest: ceil(k/4)-th largest thread value per wave, min over waves
    const int kw = (k + SNW - 1) / SNW;
    const uint32_t key = wave_sort_u32(~fkey(tval));   // descending
    const float tw = fkey_inv(~read_lane(key, kw - 1));
    if (lane == 0) sm.fred[wid] = tw;
    __syncthreads();
    float taux = sm.fred[0];
#pragma unroll
    for (int i = 1; i < SNW; ++i) taux = sm.fred[i] < taux ? sm.fred[i] : taux;
    st.flags = flags | sm.ired[0] | sm.ired[1] | sm.ired[2] | sm.ired[3];
    const float tauy = div_rn(taux, tdiv, rdiv);
    const float tc = lower_preimage(taux, tdiv, rdiv);   // x >= tc  <=>  x / t >= tauy = RN(taux / t)
    // ---- candidates: extras >= tc
#pragma unroll
    for (int r = 0; r < XPT; ++r) {
      const int i = tid + r * SNT;
      if (i < U && xr[r] >= tc && xr[r] > -__builtin_inff())
        seg_append(div_rn(xr[r], tdiv, rdiv), sm.xl_id[i], cbase, &sm);
    }
    // ---- candidates: elements >= tc of chunks whose maximum reaches tc, re-read (L2);
    // history positions are skipped (their values are the extras)
    uint32_t fm = 0u;
#pragma unroll
    for (int q = 0; q < SCPT; ++q) fm |= (cm[q] >= tc) ? (1u << q) : 0u;
    while (fm != 0u) {
      const int qa = __builtin_ctz(fm);
      fm &= fm - 1u;
      const int qb = fm != 0u ? __builtin_ctz(fm) : -1;
      if (qb >= 0) fm &= fm - 1u;
      const int64_t ca = c0 + qa * SNT + tid;
      const int64_t cb = c0 + (qb >= 0 ? qb : qa) * SNT + tid;
      const uint4 wa = (ca + 1) * EPC <= V ? rowv[ca] : load_tail_chunk<T>(rowp, ca, V);
      const uint4 wb = qb < 0 ? wa : ((cb + 1) * EPC <= V ? rowv[cb] : load_tail_chunk<T>(rowp, cb, V));
      const uint32_t ha = pen_on ? T::bits(sm.bm, qa * SNT + tid) : 0u;
      const uint32_t hb2 = pen_on ? T::bits(sm.bm, (qb >= 0 ? qb : qa) * SNT + tid) : 0u;
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        const float x = T::elem(wa, e);
        if (!((ha >> e) & 1u) && x >= tc && x > -__builtin_inff())
          seg_append(div_rn(x, tdiv, rdiv), ca * EPC + e, cbase, &sm);
      }
      if (qb >= 0) {
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          const float x = T::elem(wb, e);
          if (!((hb2 >> e) & 1u) && x >= tc && x > -__builtin_inff())
            seg_append(div_rn(x, tdiv, rdiv), cb * EPC + e, cbase, &sm);
        }
      }
    }
    __syncthreads();
    st.tau = tauy;
    st.ncand = sm.cnt;
  }
  if (tid == 0) dc_store_stat(P.stats + (int64_t)row * S + seg, st);

  // ---- arrival: the last workgroup of the row finalises it.  Every wave waits
  // for its device-coherent stores to complete before the barrier; the counter
  // increment follows them.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) sm.last = arrive_last(&P.counters[row], S);
  __syncthreads();
  if (!sm.last) return;
  if (tid == 0) __hip_atomic_store(&P.counters[row], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // ================================ finaliser ================================
  const SegStat* rs = P.stats + (int64_t)row * S;
  // wave 0 combines the per-segment statistics (S <= 64: one lane per segment)
  if (wid == 0) {
    const bool act = lane < S;
    SegStat s;
    if (act) s = dc_load_stat(rs + lane);
    const int32_t fl = wave_or(act ? s.flags : 0);
    if (greedy) {
      const float ym = act ? s.ymax : -__builtin_inff();
      const float M = wave_max_nan(ym);
      const bool nanm = M != M;
      const bool hit = act && (nanm ? (ym != ym) : (ym == M));
      const int32_t am = wave_min(hit ? s.amax : 0x7fffffff);
      if (lane == 0) {
        if (fl & SFLAG_XOVER) {
          P.status[row] = 1;   // a segment's distinct history ids outgrew its list: per-row kernel
        } else {
          put_id(P.out_ids, row, am == 0x7fffffff ? 0 : am);
          P.status[row] = 0;
          seg_write_info(P.out_info, row, PATH_GREEDY, 1, -__builtin_inff(), 0, 0, fl & 0xffff, M, am);
        }
      }
    } else {
      const float tau = wave_max(act ? s.tau : -__builtin_inff());
      const int nc = act ? s.ncand : 0;
      const bool over = ballot(act && nc > SEG_CAP) != 0ull;
      const int ncl = nc < SEG_CAP ? nc : SEG_CAP;
      const int inc = wave_incl_scan(ncl);
      if (act) sm.off[lane + 1] = inc;
      if (lane == 0) {
        sm.off[0] = 0;
        sm.fb[1] = tau;
        sm.ib[0] = fl;
        sm.ib[1] = (over || (fl & SFLAG_XOVER)) ? 1 : 0;
      }
    }
  }
  if (greedy) return;
  __syncthreads();
  const float tau = sm.fb[1];
  const int32_t sfl = sm.ib[0];
  const int32_t fl = sfl & 0xffff;
  const int total = sm.off[S];
  const float u0 = P.uniforms[row];
  const float u = (u0 >= 0.0f) ? (u0 < 1.0f ? u0 : 0x1.fffffep-1f) : 0.0f;

  auto uniform_row = [&](float Mrep) {
    // rows whose softmax is NaN: uniform 1/V over the vocabulary (sampler.py:77-80)
    const float qv = uniform_q(V);
    if (tid == 0) {
      put_id(P.out_ids, row, uniform_pick(u, qv, V));
      P.status[row] = 0;
      seg_write_info(P.out_info, row, PATH_UNIFORM, (int32_t)V, -__builtin_inff(), (int32_t)V, 0, fl, Mrep, -1);
    }
    if (P.out_probs != nullptr) {
      float* pr = P.out_probs + (int64_t)row * V;
      for (int64_t i = tid; i < V; i += SNT) pr[i] = qv;
    }
  };
  if (sfl & SFLAG_NAN) { uniform_row(__builtin_nanf("")); return; }
  if (sfl & SFLAG_PINF) { uniform_row(__builtin_inff()); return; }
  if (sm.ib[1] != 0 || total > FIN_SLOTS * SNT) {
    if (tid == 0) P.status[row] = 1;   // candidate overflow: per-row kernel
    return;
  }

  // ---- gather the candidates (each thread up to FIN_SLOTS, all loads in flight)
  float cy[FIN_SLOTS];
  int32_t cid[FIN_SLOTS];
#pragma unroll
  for (int r = 0; r < FIN_SLOTS; ++r) {
    const int f = tid + r * SNT;
    cy[r] = -__builtin_inff();
    cid[r] = 0;
    if (f < total) {
      int lo = 0, hi = S;   // segment s with off[s] <= f < off[s+1]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (sm.off[mid] <= f) lo = mid; else hi = mid;
      }
      const uint64_t e = dc_load(P.cand + ((int64_t)row * S + lo) * SEG_CAP + (f - sm.off[lo]));
      cy[r] = __uint_as_float((uint32_t)(e >> 32));
      cid[r] = (int32_t)(uint32_t)e;
    }
  }
  int nin = 0;
  float lmin = 3.40282347e38f, lmax = -__builtin_inff();
#pragma unroll
  for (int r = 0; r < FIN_SLOTS; ++r) {
    lmax = __builtin_fmaxf(lmax, cy[r]);
    if (cy[r] >= tau && cy[r] > -__builtin_inff()) { ++nin; lmin = __builtin_fminf(lmin, cy[r]); }
  }
  // row max (the maximum is always a candidate) and the count above the largest segment bound
  lmax = wave_max(lmax);
  nin = wave_sum(nin);
  lmin = wave_min(lmin);
  if (lane == 0) { sm.fred[wid] = lmax; sm.ired[wid] = nin; sm.wbase[wid] = __float_as_int(lmin); }
  __syncthreads();
  float M = sm.fred[0], lo = __int_as_float(sm.wbase[0]);
  int n1 = sm.ired[0];
#pragma unroll
  for (int w2 = 1; w2 < SNW; ++w2) {
    M = __builtin_fmaxf(M, sm.fred[w2]);
    lo = __builtin_fminf(lo, __int_as_float(sm.wbase[w2]));
    n1 += sm.ired[w2];
  }
  if (n1 == 0) { uniform_row(-__builtin_inff()); return; }   // every logit -inf
  // refine: linear histogram of [lo, M]; keep the bins up to the one holding the k-th largest
  double hist_hi = 0.0, hist_s = 0.0;
  int bstar = SHIST;   // keep everything >= tau
  if (n1 > 64 && (double)M > (double)lo) {
    hist_hi = (double)M;
    hist_s = (double)SHIST / ((double)M - (double)lo);
    for (int i = tid; i < SHIST; i += SNT) sm.hist[i] = 0u;
    if (tid == 0) sm.ib[2] = SHIST - 1;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < FIN_SLOTS; ++r)
      if (cy[r] >= tau && cy[r] > -__builtin_inff()) {
        const double t = (hist_hi - (double)cy[r]) * hist_s;
        const int bb = t <= 0.0 ? 0 : (t >= (double)(SHIST - 1) ? SHIST - 1 : (int)t);
        atomicAdd(&sm.hist[bb], 1u);
      }
    __syncthreads();
    // first bin whose inclusive count reaches k (thread t owns bin t)
    const int c = (int)sm.hist[tid];
    const int incl = wave_incl_scan(c);
    if (lane == 63) sm.ired[wid] = incl;
    __syncthreads();
    int before = 0;
#pragma unroll
    for (int w2 = 0; w2 < SNW; ++w2) before += w2 < wid ? sm.ired[w2] : 0;
    const int ci = before + incl;
    if (ci >= k && ci - c < k) sm.ib[2] = tid;
    __syncthreads();
    bstar = sm.ib[2];
  }
  // ---- compact the survivors into LDS
  if (tid == 0) sm.cnt = 0;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < FIN_SLOTS; ++r) {
    bool take = cy[r] >= tau && cy[r] > -__builtin_inff();
    if (take && bstar < SHIST) {
      const double t = (hist_hi - (double)cy[r]) * hist_s;
      const int bb = t <= 0.0 ? 0 : (t >= (double)(SHIST - 1) ? SHIST - 1 : (int)t);
      take = bb <= bstar;
    }
    const uint64_t m = ballot(take);
    if (m != 0ull) {
      int base = 0;
      const int leader = __builtin_ctzll(m);
      if (lane == leader) base = atomicAdd(&sm.cnt, __popcll(m));
      base = read_lane(base, leader);
      const int p = base + lanes_below(m);
      if (take && p < WAVE_CAP) sm.list[p] = ((uint64_t)__float_as_uint(cy[r]) << 32) | (uint32_t)cid[r];
    }
  }
  if (P.out_probs != nullptr) {
    float* pr = P.out_probs + (int64_t)row * V;
    for (int64_t i = tid; i < V; i += SNT) pr[i] = 0.0f;
  }
  __syncthreads();
  const int n2 = sm.cnt;
  if (n2 > WAVE_CAP) {
    if (tid == 0) P.status[row] = 1;   // huge tie group at the threshold: per-row kernel
    return;
  }
  if (wid != 0) return;
  if (lane == 0) P.status[row] = 0;
  const float topp = P.top_p[row];
  const bool topp_on = topp < 1.0f;
  if (n2 <= 64)
    wave_finalize<1>(sm.list, n2, k, topp_on, topp, 1.0f, 1.0f, u, row, P.out_ids, P.out_probs, V, P.out_info, fl, n1,
                     PATH_WAVE_SET);
  else if (n2 <= 128)
    wave_finalize<2>(sm.list, n2, k, topp_on, topp, 1.0f, 1.0f, u, row, P.out_ids, P.out_probs, V, P.out_info, fl, n1,
                     PATH_WAVE_SET);
  else
    wave_finalize<4>(sm.list, n2, k, topp_on, topp, 1.0f, 1.0f, u, row, P.out_ids, P.out_probs, V, P.out_info, fl, n1,
                     PATH_WAVE_SET);
}

template <typename T>
__global__ __launch_bounds__(SNT) __attribute__((amdgpu_waves_per_eu(4))) void segment_kernel(const SegParams P) {
  __shared__ SegSmem sm;
  segment_body<T>(P, sm);
}

}  // namespace ns
