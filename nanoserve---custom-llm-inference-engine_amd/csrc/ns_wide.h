// gfx950 wide path: sampled rows whose top-k is off (k <= 0 or k >= V) or larger than
// KFAST -- the rows the streaming and segment paths leave to one workgroup.  Each row is
// split over the segment kernel's 16-byte-chunk segments, so every CU works on it, and
// sampler.py:31-89 runs in up to three launches over (row, segment) workgroups, then one
// per row:
//   1. stats  (the HBM pass, the segment read twice, the second time from the L2): scaled
//      logits y (penalty sampler.py:31-38 with set semantics, temperature :40-51) -> the
//      segment's max m, finite count, NaN / +inf flags; then its histogram of counts and
//      masses exp(y - m) on the absolute grid of bins floor(64 y), the 2048 bins below
//      its max, exported.  The last segment of a row resolves NaN / +inf / all -inf rows
//      (uniform 1/V, :77-80), merges the segments' histograms (bin b below the row's top
//      bin floor(64 M) is bin b - (floor(64 M) - floor(64 m)) of a segment, its mass
//      scaled by exp(m - M)) and plans the row: without top-k and top-p it draws at once;
//      otherwise it finds the bin holding the k-th largest (:56-58) and the bins where the
//      top-p mass crosses (:60-73).
//   2. cut    (re-read): the planned bins' elements are compacted per segment, with the
//      count of those above them; each segment's mass above them is the sum of its own
//      histogram's bins (no exponential per element).
//   3. final  (one workgroup per row): orders the compacted elements (value descending,
//      id ascending) and finds the exact top-k threshold, the top-p cut as the oracle
//      defines it (float32 prefix of float32 probabilities), the kept set's mass per
//      segment, and draws: the segment holding u from the per-segment kept masses, then
//      a walk over that segment (inverse CDF in token-id order, sampler.py:84-89 against
//      a caller uniform).
//   4. probs  (only with out_probs): every token's final probability.
// A segment's masses are integer sums of exp(y - m) in units of 2^-44 and every merge
// runs in a fixed order, so every run gives the same totals.  Rows this path cannot plan
// (a k-th largest or top-p crossing more than 32 below the max, |M| of 2^18 or more, more
// planned elements than WCAND) are left to the per-row kernel (status 1).
#pragma once

#include <type_traits>

#include "ns_segment.h"

namespace ns {

constexpr int WBINS = 2048;                   // histogram bins below the row max
constexpr float WSCALE = 64.0f;               // bins per unit of scaled logit (the bins span 32 units)
constexpr int WCAND = 8192;                   // planned-bin elements one row's finaliser orders
constexpr int WIDE_MAX_ROWS = 4096;           // rows a call sends through this path
constexpr double WFX = 17592186044416.0;      // 2^44: fixed-point scale of exp(y - M) <= 1
constexpr double WFX_INV = 1.0 / 17592186044416.0;
constexpr int32_t PATH_WIDE = 7;              // out_info path code
constexpr float WMAX_PLAN = 262144.0f;         // rows with |M| at or above it (2^18: bin edges k / 64 stop
                                              // being exact floats past 2^24 / 64) are not planned

enum : int32_t { WSTEP_NONE = 0, WSTEP_CUT = 2, WSTEP_DRAWN = 3, WSTEP_UNIFORM = 4, WSTEP_FULL = 5 };

// Per-row plan and result in the workspace (128 bytes).
struct WideRow {
  float M;                 // row max of the scaled logits
  int32_t flags;           // FLAG_* and SFLAG_NAN / SFLAG_PINF
  int32_t nfin;            // finite scaled logits
  int32_t step;            // WSTEP_*
  int32_t blo, bend;       // planned bins [blo, bend]
  int32_t n_above;         // finite elements in bins < blo (from the count histogram, top-k rows)
  int32_t kon;             // top-k applies with a finite threshold (0 < k <= nfin, k < V)
  uint64_t mass_above;     // fixed-point mass of bins < blo
  uint64_t mass_tot;       // fixed-point mass of the row
  float thr;               // top-k threshold (scaled), -inf when top-k keeps every finite value
  float vstar;             // kept: y > vstar, or y == vstar and id <= istar
  int32_t istar;
  int32_t n_kept;
  double zkept;            // normaliser of the kept set
  int32_t hlen;            // the row's history length when it was planned (the probs pass reads
                           // it: a device-resident history may have grown by the drawn token)
  int32_t pad[13];
};
static_assert(sizeof(WideRow) == 128, "WideRow layout");

// Per-(row, segment) record, in the segment kernel's statistics slots (32 bytes).
struct WideSeg {
  uint64_t mass;           // pass 1: float64 bits of sum exp(y - ymax) (rows that keep every value);
                           // cut pass: its mass in bins < blo
  float ymax;              // pass 1: segment max of the finite scaled logits
  int32_t nfin;            // pass 1: finite scaled logits
  int32_t flags;           // pass 1: flags
  int32_t ncand;           // cut pass: planned-bin elements (may exceed SEG_CAP: overflow)
  int32_t nabove;          // cut pass: finite elements in bins < blo
  int32_t pad;
};
static_assert(sizeof(WideSeg) == sizeof(SegStat), "WideSeg uses the segment statistics slots");

struct WideParams {
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
  int32_t S;               // segments per row
  int32_t init_status;     // pass 1 writes status 1 for the rows it does not take
  int32_t* counters;       // [rows] arrival counters, zero between launches
  int32_t* status;         // [rows] 0 = resolved here, 1 = per-row kernel
  WideRow* rows;           // [rows]
  WideSeg* segs;           // [rows * S]
  uint64_t* shist;         // [rows * S * WBINS] pass 1: each segment's histogram below its top bin,
                           //   (count << 32) | float32 bits of the mass in units of exp(m)
  uint64_t* cand;          // [rows * S * SEG_CAP]  (float bits << 32) | token id
};

template <int NKEYS>
struct WideSmemT {
  uint32_t bm[SEG_CH * 8 / 32];              // history bitmap of one segment
  union {
    struct {
      uint32_t cnt[WBINS];
      unsigned long long mass[WBINS];
    } h;
    uint64_t keys[NKEYS];                    // the finaliser's ordered elements
  } u;
  unsigned long long segfx[MAX_SEGS];
  unsigned long long subq[MAX_SEGS];         // the finaliser's kept mass per segment
  int32_t off[MAX_SEGS + 1];
  int32_t nab[MAX_SEGS];                     // the finaliser's elements above the plan per segment
  unsigned long long ured[NWAVE];
  double dred[NWAVE];
  float fred[NWAVE];
  int32_t ired[NWAVE];
  int32_t last;
  int32_t flags;
  int32_t cnt;
  int32_t ib[8];
  float fb[4];
  double db[4];
  uint64_t kb[2];
};
using WideSmem = WideSmemT<1>;               // stats, histogram and probability passes
// The cut pass's LDS: the segment's history bitmap and the block reductions only (no
// histogram), so more of its workgroups fit a CU.
struct WideSmemLite {
  uint32_t bm[SEG_CH * 8 / 32];
  double dred[NWAVE];
  int32_t ired[NWAVE];
  int32_t flags;
  int32_t cnt;
};
using WideSmemCut = WideSmemT<WCAND>;        // the cut pass and its finaliser

// Rows this path takes: sampled (temperature != 0) and not small-k (sampler.py:55).
__host__ __device__ __forceinline__ bool wide_row(float t, int32_t k, int64_t V) { return !seg_row(t, k, V); }

// The absolute bin grid: floor(64 y), clamped far outside the plannable range (the scaling
// is exact, so the bin of a value is the same wherever it is computed).
__device__ __forceinline__ int wgrid(float y) {
  return (int)__builtin_floorf(__builtin_fminf(__builtin_fmaxf(y * WSCALE, -1.0e9f), 1.0e9f));
}
// Bin of a scaled logit below the top bin tb (= wgrid of the row's or the segment's max,
// finite; WBINS: 2048 or more bins below, or not finite).  No branch: -inf and NaN reach a
// distance past WBINS through wgrid's clamp (fmax returns the number for a NaN operand),
// +inf a negative one (tb and the clamped index lie within 1e9, so the difference does not
// overflow); the unsigned comparison sends both to WBINS.
__device__ __forceinline__ int wbin(int tb, float y) {
  const int d = tb - wgrid(y);
  return (uint32_t)d < (uint32_t)WBINS ? d : WBINS;
}
// exp(y - M) in units of 2^-44 (y <= M), truncated: (uint64_t)(e * 2^44) for the float32
// e = exp(y - M) in [0, 1] (the product with 2^44 is exact, so the integer is the same as
// through float64).  It is formed in two 32-bit halves with exact float operations:
// x = e * 2^12 (at most 4096), hi = trunc(x), lo = trunc((x - hi) * 2^32) (x - hi is exact,
// and so is the scaling); hi * 2^32 + lo = trunc(e * 2^44).
__device__ __forceinline__ uint64_t fx44(float e) {
  const float x = e * 4096.0f;
  const uint32_t hi = (uint32_t)x;
  const uint32_t lo = (uint32_t)((x - (float)hi) * 4294967296.0f);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t wfx(float M, float y) { return fx44(ns_expf(y - M)); }

// The same fixed-point mass through the hardware base-2 exponential: exp2((y - M) log2 e),
// within a few units in the last place of expf (the rounding of y - M, which both carry,
// dominates); for the histograms, whose bins only plan the row.
__device__ __forceinline__ uint64_t wfx_hw(float M, float y) {
  return fx44(__builtin_amdgcn_exp2f((y - M) * 1.4426950408889634f));
}

__device__ __forceinline__ void dc_store_wseg(WideSeg* p, const WideSeg& s) {
  const uint64_t* w = reinterpret_cast<const uint64_t*>(&s);
  uint64_t* d = reinterpret_cast<uint64_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) dc_store(d + i, w[i]);
}
__device__ __forceinline__ WideSeg dc_load_wseg(const WideSeg* p) {
  WideSeg s;
  uint64_t* w = reinterpret_cast<uint64_t*>(&s);
  const uint64_t* d = reinterpret_cast<const uint64_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = dc_load(d + i);
  return s;
}

// Block reductions over the NTH / 64 waves of a workgroup (two barriers each).
template <int NTH = SNT, typename SM>
__device__ __forceinline__ unsigned long long wsum_u64(unsigned long long v, SM* sm) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += lane_xor(v, o);
  if (lane_id() == 0) sm->ured[wave_id()] = v;
  __syncthreads();
  unsigned long long r = 0ull;
#pragma unroll
  for (int w = 0; w < NTH / 64; ++w) r += sm->ured[w];
  __syncthreads();
  return r;
}
// A 64-bit and a 32-bit block sum in one pair of barriers.
template <int NTH = SNT, typename SM>
__device__ __forceinline__ void wsum_u64_i(unsigned long long& a, int32_t& b, SM* sm) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) a += lane_xor(a, o);
  b = wave_sum(b);
  if (lane_id() == 0) { sm->ured[wave_id()] = a; sm->ired[wave_id()] = b; }
  __syncthreads();
  unsigned long long ra = 0ull;
  int32_t rb = 0;
#pragma unroll
  for (int w = 0; w < NTH / 64; ++w) { ra += sm->ured[w]; rb += sm->ired[w]; }
  __syncthreads();
  a = ra;
  b = rb;
}
// A float64 and a 32-bit block sum in one pair of barriers (the float64 terms added in the
// same order as wsum_f64).
template <int NTH = SNT, typename SM>
__device__ __forceinline__ void wsum_f64_i(double& a, int32_t& b, SM* sm) {
  a = wave_sum(a);
  b = wave_sum(b);
  if (lane_id() == 0) { sm->dred[wave_id()] = a; sm->ired[wave_id()] = b; }
  __syncthreads();
  double ra = 0.0;
  int32_t rb = 0;
#pragma unroll
  for (int w = 0; w < NTH / 64; ++w) { ra += sm->dred[w]; rb += sm->ired[w]; }
  __syncthreads();
  a = ra;
  b = rb;
}
template <int NTH = SNT, typename SM>
__device__ __forceinline__ double wsum_f64(double v, SM* sm) {
  v = wave_sum(v);
  if (lane_id() == 0) sm->dred[wave_id()] = v;
  __syncthreads();
  double r = 0.0;
#pragma unroll
  for (int w = 0; w < NTH / 64; ++w) r += sm->dred[w];
  __syncthreads();
  return r;
}
template <int NTH = SNT, typename SM>
__device__ __forceinline__ int32_t wsum_i(int32_t v, SM* sm) {
  v = wave_sum(v);
  if (lane_id() == 0) sm->ired[wave_id()] = v;
  __syncthreads();
  int32_t r = 0;
#pragma unroll
  for (int w = 0; w < NTH / 64; ++w) r += sm->ired[w];
  __syncthreads();
  return r;
}
template <int NTH = SNT, typename SM>
__device__ __forceinline__ float wmax_f(float v, SM* sm) {
  v = wave_max(v);
  if (lane_id() == 0) sm->fred[wave_id()] = v;
  __syncthreads();
  float r = sm->fred[0];
#pragma unroll
  for (int w = 1; w < NTH / 64; ++w) r = __builtin_fmaxf(r, sm->fred[w]);
  __syncthreads();
  return r;
}
// Exclusive prefix sum over the workgroup's threads; *total receives the sum.
template <int NTH = SNT, typename SM>
__device__ __forceinline__ double wexcl_f64(double v, double* total, SM* sm) {
  const double inc = wave_incl_scan(v);
  if (lane_id() == 63) sm->dred[wave_id()] = inc;
  __syncthreads();
  double off = 0.0, tot = 0.0;
#pragma unroll
  for (int w = 0; w < NTH / 64; ++w) {
    const double t = sm->dred[w];
    if (w < wave_id()) off += t;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return off + inc - v;
}
template <typename U, int NTH = SNT, typename SM>
__device__ __forceinline__ U wexcl_int(U v, U* total, SM* sm) {
  const U inc = wave_incl_scan(v);
  if (lane_id() == 63) {
    if constexpr (sizeof(U) == 8) sm->ured[wave_id()] = (unsigned long long)inc;
    else sm->ired[wave_id()] = (int32_t)inc;
  }
  __syncthreads();
  U off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NTH / 64; ++w) {
    const U t = sizeof(U) == 8 ? (U)sm->ured[w] : (U)sm->ired[w];
    if (w < wave_id()) off += t;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return off + inc - v;
}

// One row's view: parameters, the row pointer, the penalty.
struct WRowCtx {
  int row;
  int64_t V, src;
  const unsigned char* rowp;
  float tdiv, rdiv, pen, rpen, topp, u;
  float lo_t, lo_pen;   // div_lo of the temperature and of the penalty
  int32_t k, h0, H;
  bool pen_on, valid, scale, recip;
};

template <typename T>
__device__ __forceinline__ WRowCtx wide_row_ctx(const WideParams& P, int row) {
  WRowCtx c;
  c.row = row;
  c.V = P.vocab;
  const float temp = P.temperature[row];
  c.k = P.top_k[row];
  c.topp = P.top_p[row];
  c.pen = P.penalty[row];
  const float u0 = P.uniforms[row];
  c.u = (u0 >= 0.0f) ? (u0 < 1.0f ? u0 : 0x1.fffffep-1f) : 0.0f;
  c.src = P.sample_idx ? P.sample_idx[row] : (int64_t)row;
  int32_t h1 = 0;
  c.h0 = 0;
  row_history(P.hist_off, P.hist_slot, P.hist_len, P.hist_nslots, P.hist_cap, row, c.h0, h1);
  c.valid = wide_row(temp, c.k, c.V) && c.src >= 0 && c.src < P.n_rows_total && c.h0 >= 0 && h1 >= c.h0 &&
            h1 - c.h0 <= MAX_HIST;
  c.H = h1 - c.h0;
  c.pen_on = c.pen != 1.0f && c.H > 0;   // sampler.py:33
  c.tdiv = temp > 0.0f ? __builtin_fmaxf(temp, 1e-6f) : 1.0f;   // sampler.py:42
  c.rdiv = 1.0f / c.tdiv;
  c.scale = c.tdiv != 1.0f;
  c.recip = P.pen_rcp != nullptr;
  c.rpen = c.recip ? P.pen_rcp[row] : 1.0f / c.pen;
  c.lo_t = div_lo(c.tdiv, c.rdiv);
  c.lo_pen = c.recip ? __builtin_inff() : div_lo(c.pen, c.rpen);
  c.rowp = (const unsigned char*)P.logits + c.src * P.row_stride * T::SZ;
  return c;
}

// The history bitmap of elements [e0, e0 + SEG_EL) (set semantics, sampler.py:34-38),
// and sm->flags cleared.  Every thread must call it (two barriers).  Returns
// FLAG_BAD_HIST_ID when an id lies outside [0, V).  The ids are read WHB per thread at a time
// (each load instruction reads consecutive ids), so a history takes one memory round trip per
// WHB * NTH ids.
template <typename T, int NTH = SNT, typename SM>
__device__ __forceinline__ int32_t wide_bitmap(const WideParams& P, const WRowCtx& c, int64_t e0, SM* sm) {
  constexpr int SEG_EL = SEG_CH * T::EPC;
  const int tid = threadIdx.x;
  if (tid == 0) sm->flags = 0;
  if (c.pen_on)
    for (int i = tid; i < SEG_EL / 32; i += NTH) sm->bm[i] = 0u;
  __syncthreads();
  const int32_t* hp = P.hist_ids + c.h0;
  bool bad = false;
  constexpr int WHB = 8;
  for (int base = 0; c.pen_on && base < c.H; base += WHB * NTH) {
    int32_t ids[WHB];
#pragma unroll
    for (int s = 0; s < WHB; ++s) {
      const int j = base + s * NTH + tid;
      ids[s] = j < c.H ? hp[j] : 0;
    }
#pragma unroll
    for (int s = 0; s < WHB; ++s) {
      const int32_t id = ids[s];
      if (base + s * NTH + tid >= c.H) continue;
      if (id < 0 || (int64_t)id >= c.V) bad = true;
      else if ((int64_t)id >= e0 && (int64_t)id < e0 + SEG_EL) {
        const int32_t l = id - (int32_t)e0;
        atomicOr(&sm->bm[l >> 5], 1u << (l & 31));
      }
    }
  }
  if (bad) atomicOr(&sm->flags, FLAG_BAD_HIST_ID);
  __syncthreads();
  return sm->flags;
}

constexpr int WGRP = 4;   // chunks per thread per step of a segment pass

// Chunk ch of the row (past the row: -inf; the chunk holding the last tokens when V is
// not a multiple of EPC: its tokens and -inf), through the row's buffer descriptor.
template <typename T>
__device__ __forceinline__ uint4 wide_chunk_fix(const WRowCtx& c, int64_t ch, uint4 w) {
  const int64_t nfull = c.V / T::EPC;
  if (ch >= nfull) w = ch == nfull && nfull * T::EPC < c.V ? load_tail_chunk<T>(c.rowp, ch, c.V) : seg_ninf<T>();
  return w;
}

// The scaled, penalized values of chunk w (tokens id0 .. id0 + EPC - 1; -inf past V):
// sampler.py:37 then :51 in float32.  The divisions take the correctly rounded
// multiply-and-correct form; a chunk holding an operand outside its range (zero,
// huge, tiny, inf, NaN) is recomputed with IEEE divisions, one wave-uniform test per
// chunk.
template <typename T>
__device__ __forceinline__ void chunk_y_exact(const WRowCtx& c, const uint4& w, uint32_t hb, float (&y)[T::EPC]) {
#pragma unroll
  for (int e = 0; e < T::EPC; ++e) {
    float x = T::elem(w, e);
    if ((hb >> e) & 1u) x = x < 0.0f ? x * c.pen : (c.recip ? x * c.rpen : x / c.pen);
    y[e] = x / c.tdiv;
  }
}
template <typename T>
__device__ __forceinline__ void chunk_y(const WRowCtx& c, const uint4& w, uint32_t hb, int64_t id0,
                                        float (&y)[T::EPC]) {
  constexpr int EPC = T::EPC;
  bool slow = false;
#pragma unroll
  for (int e = 0; e < EPC; ++e) y[e] = T::elem(w, e);
  if (hb != 0u) {
    // history positions in this chunk (few chunks have any): the penalty per element
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      if ((hb >> e) & 1u) {
        const float x = y[e];
        if (x < 0.0f) {
          y[e] = x * c.pen;
        } else {
          // the division's multiply-and-correct form (a reciprocal penalty has lo_pen = +inf:
          // its chunks always take chunk_y_exact, which multiplies)
          const float q0 = x * c.rpen;
          const float aq = __builtin_fabsf(q0);
          slow |= !(aq >= c.lo_pen && aq <= 0x1.0p+100f);
          y[e] = __builtin_fmaf(__builtin_fmaf(-q0, c.pen, x), c.rpen, q0);
        }
      }
    }
  }
  if (c.scale) {
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const float x = y[e];
      const float q0 = x * c.rdiv;
      const float aq = __builtin_fabsf(q0);
      slow |= !(aq >= c.lo_t && aq <= 0x1.0p+100f);
      y[e] = __builtin_fmaf(__builtin_fmaf(-q0, c.tdiv, x), c.rdiv, q0);
    }
  }
  if (ballot(slow) != 0ull) {
    asm volatile("");
    if (slow) chunk_y_exact<T>(c, w, hb, y);
  }
#pragma unroll
  for (int e = 0; e < EPC; ++e)
    if (id0 + e >= c.V) y[e] = -__builtin_inff();
}

// f(y, ch) for every chunk ch = c0 + q * SNT + thread of the segment that starts inside
// the row: y the scaled, penalized values of its EPC tokens (-inf past V).  The chunks
// stream in steps of WGRP per thread, the next step's loads in flight while one step is
// processed.
struct NoHook {
  __device__ __forceinline__ void operator()(int) const {}
};
template <typename T, typename F, typename G = NoHook>
__device__ __forceinline__ void wide_chunks(const WRowCtx& c, int64_t c0, const uint32_t* bm, F&& f, G&& gend = G{}) {
  constexpr int EPC = T::EPC;
  const int tid = threadIdx.x;
  const uint32_t nbytes = (uint32_t)((c.V / EPC) * 16);
  uint4 cur[WGRP], nxt[WGRP];
#pragma unroll
  for (int j = 0; j < WGRP; ++j)
    cur[j] = buf_load16_at(c.rowp, nbytes, (uint32_t)((c0 + j * SNT) * 16), (uint32_t)tid * 16u);
#pragma unroll 1
  for (int g = 0; g < SCPT / WGRP; ++g) {
    if (g + 1 < SCPT / WGRP) {
#pragma unroll
      for (int j = 0; j < WGRP; ++j)
        nxt[j] = buf_load16_at(c.rowp, nbytes, (uint32_t)((c0 + ((g + 1) * WGRP + j) * SNT) * 16),
                               (uint32_t)tid * 16u);
    }
#pragma unroll
    for (int j = 0; j < WGRP; ++j) {
      const int lc = (g * WGRP + j) * SNT + tid;
      const int64_t ch = c0 + lc;
      if (ch * EPC < c.V) {
        float y[EPC];
        chunk_y<T>(c, wide_chunk_fix<T>(c, ch, cur[j]), c.pen_on ? T::bits(bm, lc) : 0u, ch * EPC, y);
        f(y, ch);
      }
    }
    gend(g);   // step g done (chunks g * WGRP * SNT .. + WGRP * SNT of the segment)
#pragma unroll
    for (int j = 0; j < WGRP; ++j) cur[j] = nxt[j];
  }
}

// f(y, id) for every token of the segment (ids < V only): y the scaled, penalized logit.
template <typename T, typename F>
__device__ __forceinline__ void wide_each(const WRowCtx& c, int64_t c0, const uint32_t* bm, F&& f) {
  wide_chunks<T>(c, c0, bm, [&](const float (&y)[T::EPC], int64_t ch) {
#pragma unroll
    for (int e = 0; e < T::EPC; ++e)
      if (ch * T::EPC + e < c.V) f(y[e], ch * T::EPC + e);
  });
}

// Arrival of a segment workgroup: true in the last one of its row (which resets the
// counter).  Every wave's device-coherent stores complete before the counter moves.
template <typename SM>
__device__ __forceinline__ bool wide_arrive(int32_t* counter, int S, SM* sm) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) sm->last = arrive_last(counter, S);
  __syncthreads();
  const bool last = sm->last != 0;
  if (last && threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return last;
}

// Kept-set predicate of the draw and the probabilities.
struct WKeep {
  float thr, vstar;
  int32_t istar;
  __device__ __forceinline__ bool operator()(float y, int64_t id) const {
    if (!(y > -__builtin_inff()) || !(y < __builtin_inff()) || !(y >= thr)) return false;
    return y > vstar || (y == vstar && id <= (int64_t)istar);
  }
};

// The draw inside chunks [c0, c0 + NCH): the first token (ascending id) whose cumulative
// kept probability, from pstart (the kept probability of the tokens before c0), exceeds u.
// Probabilities are float32(exp(y - M) * rz), rz = 1 / zkept in float64.  The range is
// walked in steps of NTH * WL chunks, WL consecutive chunks per thread.  When rounding
// leaves u past the range, the last token with a non-zero probability.  Every thread must
// call it.
template <typename T, int NTH, int WL, int NCH, typename SM>
__device__ __forceinline__ int64_t wide_locate(const WideParams& P, const WRowCtx& c, int64_t c0, double pstart,
                                               double rz, float M, const WKeep& keep, SM* sm, int32_t* fl) {
  constexpr int EPC = T::EPC;
  static_assert(NCH % (NTH * WL) == 0 && NCH <= SEG_CH, "whole steps inside one segment's bitmap");
  constexpr int NSTEP = NCH / (NTH * WL);
  static_assert(NSTEP * WL <= 4, "the segment's chunks of a thread fit 16 registers");
  const int tid = threadIdx.x;
  const uint32_t nbytes = (uint32_t)((c.V / EPC) * 16);
  // every step's chunks are requested first, with the history ids of the bitmap: one round
  // trip to memory for the whole walk
  uint4 raw[NSTEP][WL];
#pragma unroll
  for (int step = 0; step < NSTEP; ++step)
#pragma unroll
    for (int j = 0; j < WL; ++j)
      raw[step][j] = buf_load16_at(c.rowp, nbytes,
                                   (uint32_t)((c0 + (int64_t)step * NTH * WL + (int64_t)tid * WL + j) * 16), 0u);
  *fl |= wide_bitmap<T, NTH>(P, c, c0 * EPC, sm);
  if (tid == 0) { sm->ib[0] = 0x7fffffff; sm->ib[1] = -1; }
  const double ud = (double)c.u;
  double carry = pstart;
#pragma unroll
  for (int step = 0; step < NSTEP; ++step) {
    const int64_t cb = c0 + (int64_t)step * NTH * WL + (int64_t)tid * WL;   // first chunk of this thread
    float p[WL * EPC];
#pragma unroll
    for (int j = 0; j < WL; ++j) {
      const int64_t ch = cb + j;
      const uint4 w = wide_chunk_fix<T>(c, ch, raw[step][j]);
      const uint32_t hb = c.pen_on ? T::bits(sm->bm, (int)(ch - c0)) : 0u;
      float y[EPC];
      chunk_y<T>(c, w, hb, ch * EPC, y);
#pragma unroll
      for (int e = 0; e < EPC; ++e)
        p[j * EPC + e] = keep(y[e], ch * EPC + e) ? (float)((double)ns_expf(y[e] - M) * rz) : 0.0f;
    }
    double own = 0.0;
#pragma unroll
    for (int i = 0; i < WL * EPC; ++i) own += (double)p[i];
    double tot;
    double run = carry + wexcl_f64<NTH>(own, &tot, sm);
    int32_t first = 0x7fffffff, lastnz = -1;
#pragma unroll
    for (int i = 0; i < WL * EPC; ++i) {
      if (p[i] > 0.0f) {
        run += (double)p[i];
        const int32_t id = (int32_t)(cb * EPC + i);
        lastnz = id;
        if (run > ud && first == 0x7fffffff) first = id;
      }
    }
    if (first != 0x7fffffff) atomicMin(&sm->ib[0], first);
    if (lastnz >= 0) atomicMax(&sm->ib[1], lastnz);
    __syncthreads();
    const bool found = sm->ib[0] != 0x7fffffff;
    __syncthreads();   // every thread has read the flag before the next step may set it
    if (found) break;
    carry += tot;
  }
  int64_t tok = sm->ib[0];
  if (tok == 0x7fffffff) {
    *fl |= FLAG_LOCATE_FALLBACK;
    tok = sm->ib[1] >= 0 ? sm->ib[1] : c0 * EPC;
  }
  __syncthreads();
  return tok;
}

// A raw logit below which no token of the row reaches the scaled value B (finite): RN(x / t)
// >= B implies x >= t * B less a few units in the last place, so x >= lx for lx = RN(t * B)
// lowered by 2^-21 of itself (four units in the last place at least) and by a margin for
// subnormal quotients.  A penalty >= 1 (also as a multiply by RN(1/p) <= 1) never raises a
// value, so the bound holds for history tokens too.  -inf (no bound) for a penalty below 1 or
// an out-of-range product.
__device__ __forceinline__ float wide_raw_bound(const WRowCtx& c, float B) {
  if (!(B > -__builtin_inff()) || (c.pen_on && !(c.pen >= 1.0f))) return -__builtin_inff();
  const float L = c.scale ? B * c.tdiv : B;
  if (!(__builtin_fabsf(L) < 0x1.0p+120f)) return -__builtin_inff();
  return L - __builtin_fabsf(L) * 0x1.0p-21f - (c.tdiv + 1.0f) * 0x1.0p-140f;
}

// wide_locate for a planned row, over the tokens that can be kept: every token of the range
// whose raw logit reaches lx (a superset of the kept set, wide_raw_bound) is listed in
// ascending id order in `list` (LIST_CAP entries of (scaled value bits << 32) | id, one block
// scan of the per-thread counts, four 16-bit fields one per step), and only the listed tokens
// take the scaled value's probability and the cumulative sum.  The same tokens, values and
// probabilities as wide_locate.  Returns -2 (nothing drawn, the bitmap built) when more than
// LIST_CAP tokens reach lx: the caller then takes wide_locate.
template <typename T, int NTH, int WL, int NCH, int LIST_CAP, typename SM>
__device__ __forceinline__ int64_t wide_locate_list(const WideParams& P, const WRowCtx& c, int64_t c0, double pstart,
                                                    double rz, float M, const WKeep& keep, float lx, uint64_t* list,
                                                    SM* sm, int32_t* fl) {
  constexpr int EPC = T::EPC;
  static_assert(NCH % (NTH * WL) == 0 && NCH <= SEG_CH, "whole steps inside one segment's bitmap");
  constexpr int NSTEP = NCH / (NTH * WL);
  static_assert(NSTEP <= 4 && NSTEP * WL <= 4 && WL * EPC <= 8, "four 16-bit counts of at most 8 per thread");
  constexpr int PER = LIST_CAP / NTH;   // listed tokens per thread in the walk
  const int tid = threadIdx.x;
  const uint32_t nbytes = (uint32_t)((c.V / EPC) * 16);
  uint4 raw[NSTEP][WL];
#pragma unroll
  for (int step = 0; step < NSTEP; ++step)
#pragma unroll
    for (int j = 0; j < WL; ++j)
      raw[step][j] = buf_load16_at(c.rowp, nbytes,
                                   (uint32_t)((c0 + (int64_t)step * NTH * WL + (int64_t)tid * WL + j) * 16), 0u);
  *fl |= wide_bitmap<T, NTH>(P, c, c0 * EPC, sm);
  // the tokens reaching lx: a mask per step, their count in the step's 16-bit field
  uint32_t hit[NSTEP];
  unsigned long long cnt = 0ull;
#pragma unroll
  for (int step = 0; step < NSTEP; ++step) {
    hit[step] = 0u;
    const int64_t cb = c0 + (int64_t)step * NTH * WL + (int64_t)tid * WL;
#pragma unroll
    for (int j = 0; j < WL; ++j) {
      raw[step][j] = wide_chunk_fix<T>(c, cb + j, raw[step][j]);
#pragma unroll
      for (int e = 0; e < EPC; ++e) hit[step] |= (T::elem(raw[step][j], e) >= lx ? 1u : 0u) << (j * EPC + e);
    }
    cnt |= (unsigned long long)__popc(hit[step]) << (16 * step);
  }
  unsigned long long tot;
  const unsigned long long off = wexcl_int<unsigned long long, NTH>(cnt, &tot, sm);
  int n = 0;
#pragma unroll
  for (int step = 0; step < NSTEP; ++step) n += (int)((tot >> (16 * step)) & 0xffffu);
  if (n > LIST_CAP) return -2;   // the caller walks every token
  // the listed tokens' scaled values (chunk_y on the chunks holding one), in id order
  int before = 0;   // tokens listed by the earlier steps
#pragma unroll
  for (int step = 0; step < NSTEP; ++step) {
    const int64_t cb = c0 + (int64_t)step * NTH * WL + (int64_t)tid * WL;
    int pos = before + (int)((off >> (16 * step)) & 0xffffu);
    before += (int)((tot >> (16 * step)) & 0xffffu);
#pragma unroll
    for (int j = 0; j < WL; ++j) {
      const uint32_t hj = (hit[step] >> (j * EPC)) & ((1u << EPC) - 1u);
      if (hj != 0u) {
        const int64_t ch = cb + j;
        const uint32_t hb = c.pen_on ? T::bits(sm->bm, (int)(ch - c0)) : 0u;
        float y[EPC];
        chunk_y<T>(c, raw[step][j], hb, ch * EPC, y);
#pragma unroll
        for (int e = 0; e < EPC; ++e)
          if ((hj >> e) & 1u) list[pos++] = ((uint64_t)__float_as_uint(y[e]) << 32) | (uint32_t)(ch * EPC + e);
      }
    }
  }
  if (tid == 0) { sm->ib[0] = 0x7fffffff; sm->ib[1] = -1; }
  __syncthreads();
  // the walk over the list: PER consecutive entries per thread
  const double ud = (double)c.u;
  float p[PER];
  double own = 0.0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int li = tid * PER + i;
    p[i] = 0.0f;
    if (li < n) {
      const uint64_t e = list[li];
      const float y = __uint_as_float((uint32_t)(e >> 32));
      if (keep(y, (int32_t)(uint32_t)e)) p[i] = (float)((double)ns_expf(y - M) * rz);
    }
    own += (double)p[i];
  }
  double total;
  double run = pstart + wexcl_f64<NTH>(own, &total, sm);
  int32_t first = 0x7fffffff, lastnz = -1;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (p[i] > 0.0f) {
      const int32_t id = (int32_t)(uint32_t)list[tid * PER + i];
      run += (double)p[i];
      lastnz = id;
      if (run > ud && first == 0x7fffffff) first = id;
    }
  }
  if (first != 0x7fffffff) atomicMin(&sm->ib[0], first);
  if (lastnz >= 0) atomicMax(&sm->ib[1], lastnz);
  __syncthreads();
  int64_t tok = sm->ib[0];
  if (tok == 0x7fffffff) {
    *fl |= FLAG_LOCATE_FALLBACK;
    tok = sm->ib[1] >= 0 ? sm->ib[1] : c0 * EPC;
  }
  __syncthreads();
  return tok;
}

// (row, segment) of this workgroup: all segments of a row share blockIdx % 8 (one XCD).
__device__ __forceinline__ void wide_rowseg(int S, int* row, int* seg) {
  const int b = blockIdx.x;
  const int i8 = b >> 3;
  const int rg = i8 / S;
  *seg = i8 - rg * S;
  *row = rg * 8 + (b & 7);
}

// ------------------------------------------------------------------ the plan
// The row's plan from its histograms (8 bins per thread of the SNT threads, bin tid * 8 + j
// in hc[j], hm[j]): every thread of the last segment calls it.  Rows whose crossing lies
// past the histograms, or with more planned elements than WCAND, are left to the per-row
// kernel.
template <int BPT>
__device__ __forceinline__ void wide_plan(const WideParams& P, const WRowCtx& c, WideRow* R, int row, int32_t nfin,
                                          int32_t fl, float M, const uint32_t (&hc)[BPT],
                                          const unsigned long long (&hm)[BPT], WideSmem& sm) {
  static_assert(BPT * SNT == WBINS, "8 bins per thread");
  const int tid = threadIdx.x;
  const int64_t V = c.V;
  const bool kon0 = c.k > 0 && (int64_t)c.k < V;     // sampler.py:55
  const bool kon = kon0 && c.k <= nfin;              // otherwise the k-th largest is -inf: keep every value
  const bool pon = c.topp < 1.0f;                    // sampler.py:63
  // the row histograms' running sums
  uint32_t ccnt = 0u;
  unsigned long long cmass = 0ull;
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    ccnt += hc[j];
    cmass += hm[j];
  }
  uint32_t ctot;
  unsigned long long mtot;
  const uint32_t cbefore = wexcl_int<uint32_t>(ccnt, &ctot, &sm);
  const unsigned long long mbefore = wexcl_int<unsigned long long>(cmass, &mtot, &sm);
  const double Zt = (double)mtot * WFX_INV;

  // ---- top-k bin: the first bin where the running count reaches k
  if (tid == 0) { sm.ib[3] = WBINS; sm.ib[4] = WBINS; sm.ib[5] = WBINS; }
  __syncthreads();
  if (kon) {
    uint32_t run = cbefore;
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      const uint32_t prev = run;
      run += hc[j];
      if (prev < (uint32_t)c.k && run >= (uint32_t)c.k) sm.ib[3] = tid * BPT + j;
    }
  }
  __syncthreads();
  const int bk = kon ? sm.ib[3] : WBINS - 1;
  if (kon && bk >= WBINS) {
    // the k-th largest lies more than 32 below the max: the per-row kernel takes the row
    if (tid == 0) { P.status[row] = 1; R->step = WSTEP_NONE; }
    return;
  }
  // ---- top-p bins: the running mass crosses top_p * Z where Z lies between the mass
  // above the top-k bin and the mass through it; 1e-6 of slack on both sides
  int blo = bk, bend = bk;
  if (pon) {
    // the mass above bin bk and through it (every thread reads the owner's values)
    if (tid == bk / BPT) {
      unsigned long long m = mbefore;
#pragma unroll
      for (int j = 0; j < BPT; ++j) {
        if (tid * BPT + j == bk) { sm.db[1] = (double)m * WFX_INV; sm.db[2] = (double)(m + hm[j]) * WFX_INV; }
        m += hm[j];
      }
    }
    __syncthreads();
    const double zlo = kon ? sm.db[1] : Zt, zhi = kon ? sm.db[2] : Zt;
    const double p32 = (double)c.topp;
    const double tlo = __builtin_fmax((p32 - 1e-6) * zlo, 0.0), thi = (p32 + 1e-6) * zhi;
    unsigned long long run = mbefore;
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      const double before = (double)run * WFX_INV;
      run += hm[j];
      const double after = (double)run * WFX_INV;
      if (before <= tlo && after > tlo) atomicMin(&sm.ib[4], tid * BPT + j);
      if (before <= thi && after > thi) atomicMin(&sm.ib[5], tid * BPT + j);
    }
    __syncthreads();
    blo = sm.ib[4];
    const int bhi = sm.ib[5];
    if (blo >= WBINS || (!kon && bhi >= WBINS)) {
      // the crossing lies more than 32 below the max (or past the whole mass): per-row kernel
      if (tid == 0) { P.status[row] = 1; R->step = WSTEP_NONE; }
      return;
    }
    if (kon) {
      if (blo > bk) blo = bk;
      bend = bk;
    } else {
      bend = bhi;
    }
  }
  // elements above the planned bins and in them
  if (tid == 0) { sm.ib[6] = 0; sm.ib[7] = 0; sm.db[3] = 0.0; }
  __syncthreads();
  {
    uint32_t run = cbefore;
    unsigned long long mrun = mbefore;
    int inplan = 0;
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      const int b = tid * BPT + j;
      if (b == blo) { sm.ib[6] = (int)run; sm.segfx[0] = mrun; }
      if (b >= blo && b <= bend) inplan += (int)hc[j];
      run += hc[j];
      mrun += hm[j];
    }
    if (inplan) atomicAdd(&sm.ib[7], inplan);
  }
  __syncthreads();
  const int nplan = sm.ib[7];
  if (nplan > WCAND) {
    if (tid == 0) { P.status[row] = 1; R->step = WSTEP_NONE; }
    return;
  }
  if (tid == 0) {
    R->blo = blo;
    R->bend = bend;
    R->n_above = sm.ib[6];
    R->mass_above = sm.segfx[0];
    R->mass_tot = mtot;
    R->kon = kon ? 1 : 0;
    R->M = M;
    R->flags = fl;
    R->nfin = nfin;
    R->hlen = c.H;
    R->step = WSTEP_CUT;
  }
}


// ------------------------------------------------------------------ pass 1: stats
template <typename T>
__device__ __forceinline__ void wide_stats_body(const WideParams& P, WideSmem& sm) {
  constexpr int EPC = T::EPC;
  const int tid = threadIdx.x;
  int row, seg;
  wide_rowseg(P.S, &row, &seg);
  if (row >= P.n_sample) return;
  const WRowCtx c = wide_row_ctx<T>(P, row);
  if (!c.valid) {
    if (P.init_status && seg == 0 && tid == 0) P.status[row] = 1;
    if (seg == 0 && tid == 0) P.rows[row].step = WSTEP_NONE;
    return;
  }
  const int64_t c0 = (int64_t)seg * SEG_CH;
  int32_t flags = wide_bitmap<T>(P, c, c0 * EPC, &sm);
  // per thread: finite count, max and sum of exp(y - max) (float64, rescaled by an exact
  // float64 exp when the max moves, which a thread's first few values do)
  // (only rows that keep every finite value need the sum: the others histogram the mass
  // against the segment max below)
  const bool full_row = !(c.k > 0 && (int64_t)c.k < c.V) && !(c.topp < 1.0f);
  float mx = -__builtin_inff();
  double zt = 0.0;
  int nfin = 0;
  bool nanf = false, pinf = false;
  if (full_row) {
    wide_each<T>(c, c0, sm.bm, [&](float y, int64_t) {
      nanf |= y != y;
      pinf |= y == __builtin_inff();
      if (y > -__builtin_inff() && y < __builtin_inff()) {
        ++nfin;
        if (y > mx) {
          zt = zt * exp((double)mx - (double)y) + 1.0;
          mx = y;
        } else {
          zt += (double)ns_expf(y - mx);
        }
      }
    });
  }
  // float32 rows with a plan hold the segment in registers (chunk c0 + q * SNT + t to thread
  // t), the scaled values in place of the raw ones, for both sweeps; bfloat16 rows (twice
  // the values per register) stream it twice, the second time from the L2
  constexpr bool REGS = EPC == 4;
  uint4 v[SCPT];
  if (!full_row && !REGS) {
    wide_each<T>(c, c0, sm.bm, [&](float y, int64_t) {
      nanf |= y != y;
      pinf |= y == __builtin_inff();
      if (y > -__builtin_inff() && y < __builtin_inff()) { ++nfin; mx = __builtin_fmaxf(mx, y); }
    });
  }
  if (!full_row && REGS) {
    const uint32_t nbytes = (uint32_t)((c.V / EPC) * 16);
#pragma unroll
    for (int q = 0; q < SCPT; ++q)
      v[q] = buf_load16_at(c.rowp, nbytes, (uint32_t)((c0 + q * SNT) * 16), (uint32_t)tid * 16u);
#pragma unroll
    for (int q = 0; q < SCPT; ++q) {
      const int lc = q * SNT + tid;
      const int64_t ch = c0 + lc;
      float y[EPC];
#pragma unroll
      for (int e = 0; e < EPC; ++e) y[e] = -__builtin_inff();
      if (ch * EPC < c.V) chunk_y<T>(c, wide_chunk_fix<T>(c, ch, v[q]), c.pen_on ? T::bits(sm.bm, lc) : 0u, ch * EPC, y);
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        // branch-free: fmax passes over NaN, -inf never raises the maximum, +inf is left out
        nanf |= y[e] != y[e];
        pinf |= y[e] == __builtin_inff();
        const bool fin = __builtin_fabsf(y[e]) < __builtin_inff();
        nfin += fin ? 1 : 0;
        mx = __builtin_fmaxf(mx, y[e] < __builtin_inff() ? y[e] : -__builtin_inff());
      }
      v[q] = make_uint4(__float_as_uint(y[0]), __float_as_uint(y[1]), __float_as_uint(y[2]), __float_as_uint(y[3 % EPC]));
    }
  }
  if (ballot(nanf) != 0ull) flags |= SFLAG_NAN;
  if (ballot(pinf) != 0ull) flags |= SFLAG_PINF;
  if (lane_id() == 0 && (flags & (SFLAG_NAN | SFLAG_PINF))) atomicOr(&sm.flags, flags);
  const float smax = wmax_f(mx, &sm);
  const int32_t snfin = wsum_i(nfin, &sm);
  const double szt = wsum_f64(nfin > 0 ? zt * exp((double)mx - (double)smax) : 0.0, &sm);
  flags |= sm.flags;
  if (!full_row) {
    // the segment's histogram on the absolute grid below its top bin: counts (top-k rows)
    // and fixed-point masses exp(y - smax), from the registers; exported as (count, float32
    // mass) words for the row's planner
    for (int b = tid; b < WBINS; b += SNT) { sm.u.h.cnt[b] = 0u; sm.u.h.mass[b] = 0ull; }
    __syncthreads();
    const bool cnt_on = c.k > 0 && (int64_t)c.k < c.V;
    if (smax > -__builtin_inff() && smax < __builtin_inff()) {
      const int tb = wgrid(smax);
      auto bin_one = [&](float y) {
        const int b = wbin(tb, y);
        if (b < WBINS) {
          atomicAdd(&sm.u.h.mass[b], (unsigned long long)wfx_hw(smax, y));
          if (cnt_on) atomicAdd(&sm.u.h.cnt[b], 1u);
        }
      };
      if constexpr (REGS) {
#pragma unroll
        for (int q = 0; q < SCPT; ++q) {
          bin_one(__uint_as_float(v[q].x));
          bin_one(__uint_as_float(v[q].y));
          bin_one(__uint_as_float(v[q].z));
          bin_one(__uint_as_float(v[q].w));
        }
      } else {
        wide_each<T>(c, c0, sm.bm, [&](float y, int64_t) { bin_one(y); });
      }
    }
    __syncthreads();
    uint64_t* ex = P.shist + ((int64_t)row * P.S + seg) * WBINS;
    for (int b = tid; b < WBINS; b += SNT) {
      const float mf = (float)((double)sm.u.h.mass[b] * WFX_INV);
      dc_store(ex + b, ((uint64_t)sm.u.h.cnt[b] << 32) | __float_as_uint(mf));
    }
  }
  if (tid == 0) {
    WideSeg s{};
    s.mass = (uint64_t)__double_as_longlong(szt);
    s.ymax = smax;
    s.nfin = snfin;
    s.flags = flags;
    dc_store_wseg(P.segs + (int64_t)row * P.S + seg, s);
  }
  if (!wide_arrive(P.counters + row, P.S, &sm)) return;
  // ---- last segment of the row: M, flags, the NaN / +inf / all -inf rows
  if (wave_id() == 0) {
    const bool act = lane_id() < P.S;
    WideSeg s{};
    if (act) {
      s = dc_load_wseg(P.segs + (int64_t)row * P.S + lane_id());
      sm.u.h.mass[lane_id()] = s.mass;                                   // float64 bits of its sum
      sm.u.h.cnt[lane_id()] = __float_as_uint(s.ymax);
    }
    float M = act ? s.ymax : -__builtin_inff();
    int32_t nf = act ? s.nfin : 0, fl = act ? s.flags : 0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      M = __builtin_fmaxf(M, lane_xor(M, o));
      nf += lane_xor(nf, o);
      fl |= lane_xor(fl, o);
    }
    if (lane_id() == 0) { sm.fb[0] = M; sm.ib[0] = nf; sm.ib[1] = fl; }
    // for the merge below, once per segment (its lane): how many bins its top bin lies below
    // the row's (WBINS: no finite values, or 2048 bins or more below) and the scale exp(m - M)
    // of its masses.  Unused unless the row is planned (finite M below WMAX_PLAN).
    if (act) {
      const int ds = s.ymax > -__builtin_inff() ? wgrid(M) - wgrid(s.ymax) : WBINS;
      sm.off[lane_id()] = ds < WBINS ? ds : WBINS;
      sm.segfx[lane_id()] =
          (unsigned long long)__double_as_longlong(ds < WBINS ? exp((double)s.ymax - (double)M) : 0.0);
    }
  }
  __syncthreads();
  const float M = sm.fb[0];
  const int32_t nf = sm.ib[0], fl = sm.ib[1];
  WideRow* R = P.rows + row;
  if ((fl & (SFLAG_NAN | SFLAG_PINF)) || nf == 0) {
    // the softmax is NaN (a NaN or +inf logit, or every logit -inf): uniform 1/V
    // (sampler.py:77-80)
    const int64_t V = c.V;
    const float qv = uniform_q(V);
    if (tid == 0) {
      put_id(P.out_ids, row, uniform_pick(c.u, qv, V));
      const float mrep = (fl & SFLAG_NAN) ? __builtin_nanf("") : (nf == 0 ? -__builtin_inff() : __builtin_inff());
      seg_write_info(P.out_info, row, PATH_UNIFORM, (int32_t)V, -__builtin_inff(), (int32_t)V, 0, fl & 0xffff, mrep,
                     -1);
      P.status[row] = 0;
      R->step = WSTEP_UNIFORM;
    }
    if (P.out_probs != nullptr) {
      float* pr = P.out_probs + (int64_t)row * V;
      for (int64_t i = tid; i < V; i += SNT) pr[i] = qv;
    }
    return;
  }
  const bool kon = c.k > 0 && (int64_t)c.k < c.V && c.k <= nf;   // sampler.py:55
  const bool pon = c.topp < 1.0f;                                   // sampler.py:63
  if (!kon && !pon) {
    // ---- no top-k and no top-p: every finite value is kept.  The segments' sums rescaled to
    // the row max are the kept mass per segment; the final pass draws.
    if (tid < P.S) {
      const float ms = __uint_as_float(sm.u.h.cnt[tid]);
      const double w = ms > -__builtin_inff()
                           ? __longlong_as_double((long long)sm.u.h.mass[tid]) * exp((double)ms - (double)M)
                           : 0.0;
      WideSeg s2{};
      s2.mass = (uint64_t)__double_as_longlong(w);
      dc_store_wseg(P.segs + (int64_t)row * P.S + tid, s2);
    }
    if (tid == 0) {
      R->M = M;
      R->flags = fl;
      R->nfin = nf;
      R->hlen = c.H;
      R->step = WSTEP_FULL;
    }
    return;
  }
  if (!(__builtin_fabsf(M) < WMAX_PLAN)) {
    // bin indices of values this large are not planned: the per-row kernel takes the row
    if (tid == 0) { P.status[row] = 1; R->step = WSTEP_NONE; }
    return;
  }
  // ---- the row histograms: the segments' histograms merged onto the row's grid (bin b below
  // the row's top bin is bin b - ds of a segment whose top bin lies ds below the row's; its
  // mass in units of exp(m) scaled by exp(m - M)), in a fixed order.  Thread t merges bins
  // t + SNT * j, so each load instruction reads 512 consecutive bytes; four segments' words
  // are in flight per step (the loads of a step are issued together).  The merged bins then
  // pass through LDS to the planner's layout, 8 consecutive bins per thread.
  constexpr int BPT = WBINS / SNT;
  uint32_t hc[BPT];
  unsigned long long hm[BPT];
  {
    double acc[BPT];
#pragma unroll
    for (int j = 0; j < BPT; ++j) { acc[j] = 0.0; hc[j] = 0u; }
    constexpr int SG = 4;
    for (int sg0 = 0; sg0 < P.S; sg0 += SG) {
      uint64_t w[SG][BPT];
#pragma unroll
      for (int q = 0; q < SG; ++q) {
        const int sg = sg0 + q;
        // a segment without finite values, or 2048 bins or more below the row's top: nothing
        const int ds = sg < P.S ? sm.off[sg] : WBINS;
        const uint64_t* ex = P.shist + ((int64_t)row * P.S + sg) * WBINS;
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
          const int jj = tid + SNT * j - ds;
          w[q][j] = (ds < WBINS && jj >= 0) ? dc_load(ex + jj) : 0ull;
        }
      }
#pragma unroll
      for (int q = 0; q < SG; ++q) {
        const int sg = sg0 + q;
        const double sc = sg < P.S && sm.off[sg] < WBINS ? __longlong_as_double((long long)sm.segfx[sg]) : 0.0;
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
          acc[j] += (double)__uint_as_float((uint32_t)w[q][j]) * sc;
          hc[j] += (uint32_t)(w[q][j] >> 32);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      sm.u.h.mass[tid + SNT * j] = (unsigned long long)(acc[j] * WFX);
      sm.u.h.cnt[tid + SNT * j] = hc[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      hm[j] = sm.u.h.mass[tid * BPT + j];
      hc[j] = sm.u.h.cnt[tid * BPT + j];
    }
  }
  wide_plan<BPT>(P, c, R, row, nf, fl, M, hc, hm, sm);
}



template <typename T>
__global__ __launch_bounds__(SNT) __attribute__((amdgpu_waves_per_eu(4))) void wide_stats_kernel(const WideParams P) {
  __shared__ WideSmem sm;
  wide_stats_body<T>(P, sm);
}

// The segment kernel and the wide path's first pass in one launch over the same (row,
// segment) workgroups: greedy and small-k rows take the segment kernel's work, the others
// the stats pass (which writes status 1 for the rows neither takes).
template <typename T>
__global__ __launch_bounds__(SNT) __attribute__((amdgpu_waves_per_eu(4))) void segwide_kernel(const SegParams SP,
                                                                                            const WideParams WP) {
  __shared__ union {
    SegSmem s;
    WideSmem w;
  } sm;
  int row, seg;
  wide_rowseg(WP.S, &row, &seg);
  if (row >= WP.n_sample) return;
  if (seg_row(WP.temperature[row], WP.top_k[row], WP.vocab)) {
    if (seg == 0 && threadIdx.x == 0) WP.rows[row].step = WSTEP_NONE;   // no later wide pass for it
    segment_body<T>(SP, sm.s);
  } else {
    wide_stats_body<T>(WP, sm.w);
  }
}

// ------------------------------------------------------------------ pass 2: the planned elements
// Each segment compacts its elements in the planned bins, counts those above them, and sums
// its histogram's mass above them.
template <typename T>
__global__ __launch_bounds__(SNT) void wide_cut_kernel(const WideParams P) {
  __shared__ WideSmemLite sm;
  constexpr int EPC = T::EPC;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  int row, seg;
  wide_rowseg(P.S, &row, &seg);
  if (row >= P.n_sample) return;
  if (P.rows[row].step != WSTEP_CUT) return;
  const WRowCtx c = wide_row_ctx<T>(P, row);
  const int64_t c0 = (int64_t)seg * SEG_CH;
  WideRow* R = P.rows + row;
  const float M = R->M;
  const int TB = wgrid(M);
  const int blo = R->blo, bend = R->bend;
  const float ms = dc_load_wseg(P.segs + (int64_t)row * P.S + seg).ymax;   // this segment's max (pass 1)
  wide_bitmap<T>(P, c, c0 * EPC, &sm);
  if (tid == 0) sm.cnt = 0;
  __syncthreads();
  uint64_t* cbase = P.cand + ((int64_t)row * P.S + seg) * SEG_CAP;
  int32_t nab = 0;
  // bin b < blo  <=>  floor(64 y) > TB - blo  <=>  y >= (TB - blo + 1) / 64, and b <= bend
  // <=>  y >= (TB - bend) / 64: the grid's edges are exact floats, so two compares per
  // element classify it exactly as wbin does
  const float y_above = (float)(TB - blo + 1) * (1.0f / WSCALE);
  const float y_plan = (float)(TB - bend) * (1.0f / WSCALE);
  wide_chunks<T>(c, c0, sm.bm, [&](const float (&y)[EPC], int64_t ch) {
    bool any = false;
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      nab += y[e] >= y_above ? 1 : 0;
      any |= y[e] >= y_plan && y[e] < y_above;
    }
    // the planned elements of the chunk, appended wave-aggregated (one test per chunk)
    if (ballot(any) != 0ull) {
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        const bool take = y[e] >= y_plan && y[e] < y_above;
        const uint64_t m = ballot(take);
        if (m != 0ull) {
          const int leader = __builtin_ctzll(m);
          int base = 0;
          if (lane == leader) base = atomicAdd(&sm.cnt, __popcll(m));
          base = read_lane(base, leader);
          const int pos = base + lanes_below(m);
          if (take && pos < SEG_CAP)
            dc_store(cbase + pos, ((uint64_t)__float_as_uint(y[e]) << 32) | (uint32_t)(ch * EPC + e));
        }
      }
    }
  });
  // the mass above the plan: this segment's histogram bins below row bin blo (its bin jj is
  // row bin jj + ds), in units of exp(ms), scaled to exp(M)
  double part = 0.0;
  if (ms > -__builtin_inff()) {
    const int ds = TB - wgrid(ms);
    const uint64_t* ex = P.shist + ((int64_t)row * P.S + seg) * WBINS;
    const int lim = blo - ds < WBINS ? blo - ds : WBINS;
    for (int jj = tid; jj < lim; jj += SNT) part += (double)__uint_as_float((uint32_t)dc_load(ex + jj));
  }
  int32_t snab = nab;
  wsum_f64_i(part, snab, &sm);
  const double above = part * (ms > -__builtin_inff() ? exp((double)ms - (double)M) : 0.0);
  if (tid == 0) {
    WideSeg s{};
    s.mass = (uint64_t)(above * WFX);
    s.ncand = sm.cnt;
    s.nabove = snab;
    dc_store_wseg(P.segs + (int64_t)row * P.S + seg, s);
  }
}

// Ascending bitonic sort of the keys at positions [0, P2) of the workgroup, E per thread in
// registers (position tid * E + j in k[j]); P2 a power of two with 64 * E <= P2 <= NT * E.
// Compare-exchanges at a distance below E stay inside a thread, those below 64 * E go
// between the lanes of a wave (DPP / permlane, no LDS), the longer ones through `buf`
// (P2 keys of LDS, stored j-major so every exchange reads and writes consecutive
// addresses).  Every thread must call it.
template <int E>
__device__ __forceinline__ void block_sort_regs(uint64_t (&k)[E], int P2, uint64_t* buf) {
  // Every compare-exchange keeps the smaller key where flip is 0 and the larger where it is
  // all ones, comparing the keys xored with flip: the direction never becomes a lane mask
  // of its own (which the compiler would combine with the comparison on the scalar unit).
  const int t = threadIdx.x;
  const int lane = lane_id();
  const bool act = t * E < P2;
  for (int size = 2; size <= P2; size <<= 1) {
    const bool asc_t = ((t * E) & size) == 0;
    for (int stride = size >> 1; stride >= 64 * E; stride >>= 1) {
      if (act) {
#pragma unroll
        for (int j = 0; j < E; ++j) buf[j * NT + t] = k[j];
      }
      __syncthreads();
      if (act) {
        const int pt = t ^ (stride / E);
        const uint64_t flip = (((t & (stride / E)) == 0) == asc_t) ? 0ull : ~0ull;
#pragma unroll
        for (int j = 0; j < E; ++j) {
          const uint64_t o = buf[j * NT + pt];
          k[j] = (o ^ flip) < (k[j] ^ flip) ? o : k[j];
        }
      }
      __syncthreads();
    }
    if (act) {
#pragma unroll
      for (int ls = 5; ls >= 0; --ls) {
        if ((E << ls) < size) {
          const uint64_t flip = (((lane & (1 << ls)) == 0) == asc_t) ? 0ull : ~0ull;
#pragma unroll
          for (int j = 0; j < E; ++j) {
            const uint64_t o = lane_xor(k[j], 1 << ls);
            k[j] = (o ^ flip) < (k[j] ^ flip) ? o : k[j];
          }
        }
      }
#pragma unroll
      for (int s = E / 2; s >= 1; s >>= 1) {
        if (s < size) {
#pragma unroll
          for (int j = 0; j < E; ++j) {
            if ((j & s) == 0) {
              const uint64_t flip = (((t * E + j) & size) == 0) ? 0ull : ~0ull;
              const uint64_t a = k[j], b = k[j + s];
              const bool sw = (b ^ flip) < (a ^ flip);
              k[j] = sw ? b : a;
              k[j + s] = sw ? a : b;
            }
          }
        }
      }
    }
  }
}

// The key at position pos of the keys held E per thread (a block broadcast, one barrier;
// `slot` must not be read by another broadcast in flight).
template <int E, typename SM>
__device__ __forceinline__ uint64_t block_key_at(const uint64_t (&k)[E], int pos, uint64_t* slot, SM*) {
  const int p0 = (int)threadIdx.x * E;
  if (pos >= p0 && pos < p0 + E) {
#pragma unroll
    for (int j = 0; j < E; ++j)
      if (p0 + j == pos) *slot = k[j];
  }
  __syncthreads();
  return *slot;
}

// ------------------------------------------------------------------ pass 3b: the row's cut and draw
// One 1024-thread workgroup per planned row: the planned elements ordered in LDS (value
// descending, id ascending), the exact top-k threshold and top-p cut, the kept mass per
// segment, the draw.
template <typename T>
__device__ __forceinline__ void wide_final_row(const WideParams& P, WideSmemCut& sm, const int row) {
  constexpr int EPC = T::EPC;
  constexpr int SEG_EL = SEG_CH * EPC;
  const int tid = threadIdx.x;
  if (row >= P.n_sample) return;
  WideRow* R = P.rows + row;
  const int32_t step = R->step;
  if (step != WSTEP_CUT && step != WSTEP_FULL) return;
  // every segment's record (one lane of wave 0 each), requested ahead of the row's parameters
  WideSeg sg{};
  if (tid < P.S) sg = dc_load_wseg(P.segs + (int64_t)row * P.S + tid);
  const WRowCtx c = wide_row_ctx<T>(P, row);
  const float M = R->M;
  int32_t fl = R->flags & 0xffff;
  const int32_t nfin = R->nfin;
  if (step == WSTEP_FULL) {
    // ---- every finite value kept: the segment holding u from the per-segment masses, then
    // the walk inside it (the masses read in parallel, then summed in segment order)
    if (tid < P.S) sm.subq[tid] = sg.mass;
    __syncthreads();
    if (tid == 0) {
      double Z = 0.0;
      for (int i = 0; i < P.S; ++i) Z += __longlong_as_double((long long)sm.subq[i]);
      const double ud = (double)c.u * Z;
      double run = 0.0, start = 0.0, laststart = 0.0;
      int s = -1, lastnz = -1;
      for (int i = 0; i < P.S; ++i) {
        const double w = __longlong_as_double((long long)sm.subq[i]);
        if (w > 0.0) { lastnz = i; laststart = run; }
        if (s < 0 && run + w > ud && w > 0.0) { s = i; start = run; }
        run += w;
      }
      if (s < 0) { s = lastnz >= 0 ? lastnz : 0; start = laststart; }
      sm.ib[2] = s;
      sm.db[0] = start / Z;
      sm.db[3] = Z;
    }
    __syncthreads();
    const int s = sm.ib[2];
    const double start = sm.db[0], Z = sm.db[3];
    const WKeep keep{-__builtin_inff(), -__builtin_inff(), 0x7fffffff};
    // two consecutive float32 chunks per thread a step, as for the planned rows below
    const int64_t tok =
        wide_locate<T, NT, EPC == 4 ? 2 : 1, SEG_CH>(P, c, (int64_t)s * SEG_CH, start, 1.0 / Z, M, keep, &sm, &fl);
    if (tid == 0) {
      put_id(P.out_ids, row, tok);
      seg_write_info(P.out_info, row, PATH_WIDE, nfin, -__builtin_inff(), nfin, 0, fl, -__builtin_inff(), -1);
      R->thr = -__builtin_inff();
      R->vstar = -__builtin_inff();
      R->istar = 0x7fffffff;
      R->n_kept = nfin;
      R->zkept = Z;
      R->step = WSTEP_DRAWN;
      P.status[row] = 0;
    }
    return;
  }
  const bool kon = R->kon != 0;
  const bool pon = c.topp < 1.0f;
  const bool kon0 = c.k > 0 && (int64_t)c.k < c.V;
  if (wave_id() == 0) {
    // the segments' candidate offsets (their counts capped at SEG_CAP, a prefix over the lanes:
    // S <= 64, one lane per segment), the overflow flag and the elements above the plan
    const int l = lane_id();
    const bool act = l < P.S;
    const int cnt = act ? sg.ncand : 0;
    const int capped = cnt < SEG_CAP ? cnt : SEG_CAP;
    const int incl = wave_incl_scan(capped);
    const bool over = ballot(act && cnt > SEG_CAP) != 0ull;
    const int o = read_lane(incl, 63);
    const int nab = wave_sum(act ? sg.nabove : 0);
    if (act) {
      sm.segfx[l] = sg.mass;
      sm.subq[l] = sg.mass;   // the kept mass per segment starts from the mass above the plan
      sm.off[l] = incl - capped;
      sm.nab[l] = sg.nabove;
    }
    if (l == 0) {
      sm.off[P.S] = o;
      sm.ib[0] = over || o > WCAND;
      sm.ib[3] = nab;
    }
  }
  __syncthreads();
  // finite elements above the planned bins: the compaction pass's counts (top-p rows do not
  // histogram counts)
  const int32_t n_above = sm.ib[3];
  // the mass above the planned bins: the segments' sums from the compaction pass (the same
  // fixed-point terms the histogram holds when it holds masses)
  uint64_t mass_above = 0ull;
  for (int i = 0; i < P.S; ++i) mass_above += sm.segfx[i];
  const int n = sm.off[P.S];
  if (sm.ib[0] || n == 0) {
    if (tid == 0) { P.status[row] = 1; R->step = WSTEP_NONE; }
    return;
  }
  // the planned elements as sort keys (value descending, id ascending), EPT per thread in
  // registers at positions tid * EPT + j, ordered over a power of two of positions; EPT the
  // fewest keys per thread that hold them all (a handful of planned elements is ordered
  // inside one wave).  Thread t first holds elements j * NT + t (each load instruction reads
  // consecutive words): with more than one key per thread the sorted range is every position
  // (n > NT * EPT / 2), and with one it is the first next_pow2(n) >= n threads.
  auto tail = [&](auto ept) {
    constexpr int EPT = decltype(ept)::value;
    const int p0 = tid * EPT;
    uint64_t kk[EPT];
    {
      int s = 0;
  #pragma unroll
      for (int j = 0; j < EPT; ++j) {
        const int i = j * NT + tid;
        kk[j] = ~0ull;
        if (i < n) {
          while (s + 1 < P.S && sm.off[s + 1] <= i) ++s;
          const uint64_t e = dc_load(P.cand + ((int64_t)row * P.S + s) * SEG_CAP + (i - sm.off[s]));
          kk[j] = desc_key(__uint_as_float((uint32_t)(e >> 32)), (uint32_t)e);
        }
      }
    }
    int P2 = next_pow2(n < 2 ? 2 : n);
    if (P2 < 64 * EPT) P2 = 64 * EPT;
    block_sort_regs<EPT>(kk, P2, sm.u.keys);
    // ---- top-k threshold: the k-th largest, k - 1 - n_above places into the ordered elements
    float thr = -__builtin_inff();
    if (kon) {
      const int r = c.k - 1 - n_above;
      if (r < 0 || r >= n) {
        if (tid == 0) { P.status[row] = 1; R->step = WSTEP_NONE; }
        return;
      }
      thr = desc_key_val(block_key_at<EPT>(kk, r, &sm.kb[0], &sm));
    }
    // per element: kept by top-k, its mass, its float32 probability under the top-k set
    // (without top-k every planned element, all finite, is a top-k element, and the top-k
    // mass is not used: the row-uniform branch skips both block sums)
    unsigned long long mtopk = 0ull;
    int32_t n_topk_c = n;
    if (kon) {
      unsigned long long mk = 0ull;
      int nk_own = 0;
  #pragma unroll
      for (int j = 0; j < EPT; ++j) {
        if (p0 + j < n) {
          const float y = desc_key_val(kk[j]);
          if (y >= thr) { mk += wfx(M, y); ++nk_own; }
        }
      }
      wsum_u64_i<NT>(mk, nk_own, &sm);
      mtopk = mk;
      n_topk_c = nk_own;
    }
    const int32_t n_topk = kon ? n_above + n_topk_c : nfin;
    const uint64_t zk_fx = kon ? mass_above + mtopk : R->mass_tot;
    const double zk = (double)zk_fx * WFX_INV;
    const double rzk = 1.0 / zk;
    // ---- top-p: first position whose float32 prefix of float32 probabilities exceeds top_p
    int J = n_topk_c - 1;          // without top-p: every top-k element is kept
    if (pon) {
      const double base = (double)mass_above * WFX_INV * rzk;
      if (n_above > 0 && (float)base > c.topp) {
        if (tid == 0) { P.status[row] = 1; R->step = WSTEP_NONE; }
        return;
      }
      float qv[EPT];
      double qs = 0.0;
  #pragma unroll
      for (int j = 0; j < EPT; ++j) {
        qv[j] = 0.0f;
        if (p0 + j < n) {
          const float y = desc_key_val(kk[j]);
          if (y >= thr) qv[j] = (float)((double)ns_expf(y - M) * rzk);
        }
        qs += (double)qv[j];
      }
      double tot;
      if (tid == 0) sm.ib[1] = 0x7fffffff;   // ordered before the atomics below by the scan's barriers
      double run = base + wexcl_f64<NT>(qs, &tot, &sm);
      int cross = 0x7fffffff;
  #pragma unroll
      for (int j = 0; j < EPT; ++j) {
        const int pos = p0 + j;
        if (pos < n && pos < n_topk_c) {
          run += (double)qv[j];
          if ((float)run > c.topp && cross == 0x7fffffff) cross = pos;
        }
      }
      if (cross != 0x7fffffff) atomicMin(&sm.ib[1], cross);
      __syncthreads();
      cross = sm.ib[1];
      if (cross != 0x7fffffff) {
        J = cross;
      } else if (!kon0) {
        // top-p alone and no crossing among the planned elements: the plan missed it
        if (tid == 0) { P.status[row] = 1; R->step = WSTEP_NONE; }
        return;
      }
    }
    if (J < 0) J = 0;
    const uint64_t kc = block_key_at<EPT>(kk, J, &sm.kb[1], &sm);
    const float vstar = pon ? desc_key_val(kc) : -__builtin_inff();
    const int32_t istar = pon ? (int32_t)desc_key_id(kc) : 0x7fffffff;
    const int32_t n_kept = pon ? n_above + J + 1 : n_topk;
    const WKeep keep{thr, vstar, istar};
    // ---- kept mass per segment: above the planned bins plus the kept planned elements
    unsigned long long mkept = 0ull;
  #pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int pos = p0 + j;
      if (pos < n && pos <= J) {
        const float y = desc_key_val(kk[j]);
        if (y >= thr) {
          const uint64_t fx = wfx(M, y);
          mkept += fx;
          atomicAdd(&sm.subq[desc_key_id(kk[j]) / SEG_EL], (unsigned long long)fx);
        }
      }
    }
    const unsigned long long mk2 = wsum_u64<NT>(mkept, &sm);
    const uint64_t zkept_fx = pon ? mass_above + mk2 : zk_fx;
    const double zkept = (double)zkept_fx * WFX_INV;
    if (wave_id() == 0) {
      // the segment holding u, from the kept mass per segment (S <= 64: one lane each, a
      // prefix over the lanes): the first segment with kept mass whose end passes u, else the
      // last with kept mass
      const int l = lane_id();
      const bool act = l < P.S;
      const uint64_t q = act ? sm.subq[l] : 0ull;
      const double p = act ? (double)q * WFX_INV * (1.0 / zkept) : 0.0;
      const double incl = wave_incl_scan(p);
      const double ud = (double)c.u;
      const uint64_t nz = ballot(act && q != 0ull);
      const uint64_t hit = ballot(act && q != 0ull && incl > ud);
      const int s = hit != 0ull ? __builtin_ctzll(hit) : (nz != 0ull ? 63 - __builtin_clzll(nz) : 0);
      const double start = read_lane(incl - p, s);
      if (l == 0) {
        sm.ib[2] = s;
        sm.db[0] = start;
      }
    }
    __syncthreads();
    const int s = sm.ib[2];
    const double start = sm.db[0];
    // the walk over that segment: two consecutive float32 chunks per thread a step (one
    // bfloat16 chunk: the same registers)
    constexpr int WL = EPC == 4 ? 2 : 1;
    // Float32 segments whose elements above the plan and planned elements together fit the
    // sort's LDS keys (free now) list the tokens that can be kept there; a segment holding more
    // (a long nucleus) walks every token, and so do bfloat16 rows (the listed walk's registers
    // beside the wider chunks spill there).
    int64_t tok = -2;
    if (EPC == 4 && sm.nab[s] + (sm.off[s + 1] - sm.off[s]) <= WCAND) {
      const float lx = wide_raw_bound(c, __builtin_fmaxf(thr, vstar));
      tok = wide_locate_list<T, NT, WL, SEG_CH, WCAND>(P, c, (int64_t)s * SEG_CH, start, 1.0 / zkept, M, keep, lx,
                                                       sm.u.keys, &sm, &fl);
    }
    if (tok == -2) tok = wide_locate<T, NT, WL, SEG_CH>(P, c, (int64_t)s * SEG_CH, start, 1.0 / zkept, M, keep, &sm, &fl);
    if (tid == 0) {
      put_id(P.out_ids, row, tok);
      seg_write_info(P.out_info, row, PATH_WIDE, n_kept, kon0 ? thr : -__builtin_inff(), n_topk, n, fl, vstar, istar);
      R->thr = thr;
      R->vstar = vstar;
      R->istar = istar;
      R->n_kept = n_kept;
      R->zkept = zkept;
      R->step = WSTEP_DRAWN;
      P.status[row] = 0;
    }

  };
  if (n <= NT) tail(std::integral_constant<int, 1>{});
  else if (n <= 2 * NT) tail(std::integral_constant<int, 2>{});
  else if (n <= 4 * NT) tail(std::integral_constant<int, 4>{});
  else tail(std::integral_constant<int, WCAND / NT>{});
}

// ------------------------------------------------------------------ pass 4: probabilities
template <typename T>
__global__ __launch_bounds__(SNT) void wide_probs_kernel(const WideParams P) {
  __shared__ WideSmem sm;
  constexpr int EPC = T::EPC;
  int row, seg;
  wide_rowseg(P.S, &row, &seg);
  if (row >= P.n_sample) return;
  const WideRow* R = P.rows + row;
  if (R->step != WSTEP_DRAWN) return;
  WRowCtx c = wide_row_ctx<T>(P, row);
  c.H = R->hlen;                             // the history the row was sampled with
  c.pen_on = c.pen != 1.0f && c.H > 0;
  const int64_t c0 = (int64_t)seg * SEG_CH;
  wide_bitmap<T>(P, c, c0 * EPC, &sm);
  const float M = R->M;
  const double rz = 1.0 / R->zkept;
  const WKeep keep{R->thr, R->vstar, R->istar};
  float* pr = P.out_probs + (int64_t)row * c.V;
  wide_each<T>(c, c0, sm.bm, [&](float y, int64_t id) {
    pr[id] = keep(y, id) ? (float)((double)ns_expf(y - M) * rz) : 0.0f;
  });
}

}  // namespace ns
