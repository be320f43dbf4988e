// gfx950 token sampler: kernel body and the C-ABI entry points.
// Design notes are in ns_sample_kernel.h; the ABI is declared in
// include/ns_sampling.h.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "ns_sample_kernel.h"
#include "ns_segment.h"
#include "ns_wide.h"
#include "ns_lmhead.h"
#include "ns_rng.h"
#include "ns_sampling.h"

static_assert(ns::WIDE_MAX_ROWS == NS_WIDE_MAX_ROWS, "wide-path row limit");
static_assert(ns::MAX_HIST == NS_MAX_HISTORY, "per-row history limit");
static_assert(ns::LDS_HIST == NS_LDS_HISTORY, "history kept in LDS by the general code");

namespace ns {

constexpr float NEG_INF = -__builtin_inff();
constexpr float POS_INF = __builtin_inff();
constexpr float FLT_MAXV = 3.40282347e38f;

template <typename T>
__device__ __forceinline__ uint4 ninf_chunk() {
  const uint32_t w = T::EPC == 8 ? 0xff80ff80u : 0xff800000u;
  return make_uint4(w, w, w, w);
}

// Wave-aggregated append of (x, id) into the LDS candidate array.  Must be
// reached by all lanes of the wave (convergent control flow); `take` selects.
__device__ __forceinline__ void cand_append(bool take, float x, int64_t id, uint64_t* cand, Misc* misc) {
  take = take && x > -__builtin_inff();   // -inf entries (history positions of the chunk layout) never enter
  uint64_t m = ballot(take);
  if (m == 0ull) return;
  int leader = __builtin_ctzll(m);
  int base = 0;
  if (lane_id() == leader) base = atomicAdd(&misc->cand_n, __popcll(m));
  base = __shfl(base, leader);
  int pos = base + lanes_below(m);
  if (take && pos < CAP) cand[pos] = ((uint64_t)__float_as_uint(x) << 32) | (uint32_t)id;
}

// Streaming visit of this row thread's chunks (history positions read as -inf).
// f(x, id, j) with j the chunk row.
template <typename T, typename F>
__device__ __forceinline__ void visit_rows(const uint4* rowv, const uint32_t* bm, bool pen_on, int64_t nch,
                                           int64_t nrows_j, F&& f) {
  const int tid = threadIdx.x;
  for (int64_t j = 0; j < nrows_j; j += 4) {
    uint4 v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      int64_t c = (j + q) * RT + tid;
      v[q] = (j + q < nrows_j && c < nch) ? rowv[c] : ninf_chunk<T>();
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      int64_t c = (j + q) * RT + tid;
      if (j + q < nrows_j && c < nch) {
        uint4 w = v[q];
        if (pen_on) w = T::mask(w, T::bits(bm, c));
#pragma unroll
        for (int e = 0; e < T::EPC; ++e) f(T::elem(w, e), c * T::EPC + e, j + q);
      }
    }
  }
}

// Linear-bin histogram levels used by the generic paths.  Level r maps a value
// v with hi_r >= v to bin (hi_r - v) * s_r clamped to [0, NB-1]; membership in
// level r+1 is "bin at every earlier level equals the chosen bin".
struct Levels {
  double hi[MAX_LEVELS];
  double s[MAX_LEVELS];
  int b[MAX_LEVELS];
  int n;
  __device__ __forceinline__ static int bin(double hi, double s, float v) {
    double t = (hi - (double)v) * s;
    int b = t <= 0.0 ? 0 : (t >= (double)(NB - 1) ? NB - 1 : (int)t);
    return b;
  }
  // h, sc, bb and r are block-uniform: the fields are taken from the first lane so they
  // live in scalar registers
  __device__ __forceinline__ void set(int r, double h, double sc, int bb) {
    const double hu = uniform_f64(h), su = uniform_f64(sc);
    const int bu = __builtin_amdgcn_readfirstlane(bb);
#pragma unroll
    for (int i = 0; i < MAX_LEVELS; ++i)
      if (i == r) { hi[i] = hu; s[i] = su; b[i] = bu; }
    n = r + 1;
  }
  __device__ __forceinline__ bool member(float v) const {
    bool ok = true;
#pragma unroll
    for (int r = 0; r < MAX_LEVELS; ++r)
      if (r < n) ok = ok && bin(hi[r], s[r], v) == b[r];
    return ok;
  }
};

// Find the first bin whose inclusive cumulative (count or fixed-point mass)
// exceeds `target` (strictly greater if `strict`, else >=).  Thread t owns bins
// 2t and 2t+1.  Returns the bin (or -1) and the cumulative before it.
__device__ __forceinline__ int find_bin(const uint64_t* vals64, const uint32_t* vals32, bool use64, double target,
                                        bool strict, double* before, Misc* misc) {
  const int t = threadIdx.x;
  double a = use64 ? (double)vals64[2 * t] : (double)vals32[2 * t];
  double b = use64 ? (double)vals64[2 * t + 1] : (double)vals32[2 * t + 1];
  double tot;
  if (t == 0) { misc->ib[10] = -1; }
  double pre = block_excl_scan(a + b, &tot, &misc->red);  // contains barriers
  auto over = [&](double c) { return strict ? (c > target) : (c >= target); };
  if (!over(pre) && over(pre + a)) { misc->ib[10] = 2 * t; misc->db[6] = pre; }
  else if (!over(pre + a) && over(pre + a + b)) { misc->ib[10] = 2 * t + 1; misc->db[6] = pre + a; }
  __syncthreads();
  int r = misc->ib[10];
  *before = misc->db[6];
  __syncthreads();
  return r;
}

// Threshold tau with count(values >= tau) >= k from per-thread value arrays
// (chunk or group maxima): histogram over [lo, hi], first bin reaching k, tau =
// the smallest value in bins up to it.  Returns -inf when fewer than k values.
template <int NV>
__device__ __forceinline__ float select_tau(const float (&v)[NV], bool active, int k, uint32_t* hcnt, Misc* misc) {
  float hi = NEG_INF, lo = POS_INF;
  int cnt = 0;
  if (active) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (v[i] > NEG_INF) { hi = __builtin_fmaxf(hi, v[i]); lo = __builtin_fminf(lo, v[i]); ++cnt; }
  }
  hi = block_max_nan(hi, &misc->red);
  lo = block_min_nan(lo, &misc->red);
  int64_t total = block_sum_i64(cnt, &misc->red);
  if (total < k) return NEG_INF;
  if (!(hi > lo)) return lo;
  const double dh = hi, ds = (double)NB / ((double)hi - (double)lo);
  for (int i = threadIdx.x; i < NB; i += NT) hcnt[i] = 0u;
  __syncthreads();
  if (active) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (v[i] > NEG_INF) atomicAdd(&hcnt[Levels::bin(dh, ds, v[i])], 1u);
  }
  __syncthreads();
  double before;
  int bstar = find_bin(nullptr, hcnt, false, (double)k, false, &before, misc);
  float m = POS_INF;
  if (active) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (v[i] > NEG_INF && Levels::bin(dh, ds, v[i]) <= bstar) m = __builtin_fminf(m, v[i]);
  }
  return block_min_nan(m, &misc->red);
}

struct RowOut {
  IdSink out_ids;
  float* out_probs;
  int32_t* out_info;
  int row;
  int64_t V;
};

__device__ __forceinline__ void write_info(const RowOut& o, int32_t path, int32_t n_kept, float thr, int32_t n_topk,
                                           int32_t n_cand, int32_t flags, float vstar, int32_t istar) {
  if (o.out_info == nullptr || threadIdx.x != 0) return;
  int32_t* w = o.out_info + (int64_t)o.row * INFO_WORDS;
  w[0] = path; w[1] = n_kept; w[2] = (int32_t)__float_as_uint(thr); w[3] = n_topk;
  w[4] = n_cand; w[5] = flags; w[6] = (int32_t)__float_as_uint(vstar); w[7] = istar;
}

__device__ __forceinline__ void zero_probs(const RowOut& o) {
  if (o.out_probs == nullptr) return;
  float* pr = o.out_probs + (int64_t)o.row * o.V;
  for (int64_t i = threadIdx.x; i < o.V; i += NT) pr[i] = 0.0f;
  __syncthreads();
}

// Exact selection, top-p and draw over the n entries (x, id) in `cand`.
// need_topk: keep the entries >= the k-th largest scaled value; need_topp: apply
// the nucleus cut.  Without either, the entries are the whole kept set.
__device__ __attribute__((always_inline)) inline void lds_set(int n, bool need_topk, int k, bool need_topp, float p32, float My, float tdiv, float rdiv,
                        float u, uint64_t* cand, Misc* misc, const RowOut& o, int32_t path, int32_t flags,
                        float thr_in, int32_t n_topk_in) {
  const int tid = threadIdx.x;
  uint64_t kv[CAP / NT];
#pragma unroll
  for (int q = 0; q < CAP / NT; ++q) {
    int i = tid + q * NT;
    kv[q] = ~0ull;
    if (i < n) {
      uint64_t e = cand[i];
      float x = __uint_as_float((uint32_t)(e >> 32));
      float y = div_rn(x, tdiv, rdiv);
      kv[q] = desc_key(y, (uint32_t)e);
    }
  }
  const int P = next_pow2(n < 2 ? 2 : n);
  if (tid == 0) { misc->ib[1] = n; misc->ib[2] = -1; misc->ib[3] = -1; }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < CAP / NT; ++q) {
    int i = tid + q * NT;
    if (i < P) cand[i] = kv[q];
  }
  __syncthreads();
  lds_bitonic_sort(cand, P);

  // top-k: keep every entry >= the k-th largest (ties kept, sampler.py:56-58)
  int nk = n;
  float thr = thr_in;
  if (need_topk) {
    if (n < k) {
      // fewer than k finite candidates: the k-th largest is -inf and nothing is removed
      thr = NEG_INF;
    } else {
      thr = desc_key_val(cand[k - 1]);
      for (int i = tid; i < n; i += NT) {
        float yi = desc_key_val(cand[i]);
        if (yi >= thr && (i + 1 == n || desc_key_val(cand[i + 1]) < thr)) misc->ib[1] = i + 1;
      }
      __syncthreads();
      nk = misc->ib[1];
    }
  }
  const int n_topk = need_topk ? nk : n_topk_in;

  // masses over sorted positions; thread t owns positions 4t .. 4t+3
  const int p0 = tid * (CAP / NT);
  float e[CAP / NT];
  double es = 0.0;
#pragma unroll
  for (int q = 0; q < CAP / NT; ++q) {
    int pos = p0 + q;
    e[q] = pos < nk ? ns_expf(desc_key_val(cand[pos]) - My) : 0.0f;
    es += (double)e[q];
  }
  int nf = nk;
  float vstar = NEG_INF;
  int32_t istar = -1;
  if (need_topp) {
    // sampler.py:64-73: sorted softmax, float32 prefix sums, keep through the crossing
    double Z = block_sum(es, &misc->red);
    float qv[CAP / NT];
    double qs = 0.0;
#pragma unroll
    for (int q = 0; q < CAP / NT; ++q) {
      qv[q] = (p0 + q) < nk ? (float)((double)e[q] / Z) : 0.0f;
      qs += (double)qv[q];
    }
    double tot;
    double run = block_excl_scan(qs, &tot, &misc->red);
#pragma unroll
    for (int q = 0; q < CAP / NT; ++q) {
      int pos = p0 + q;
      if (pos < nk) {
        float cprev = (float)run;
        run += (double)qv[q];
        float c = (float)run;
        if (c > p32 && (pos == 0 || !(cprev > p32))) misc->ib[2] = pos;
      }
    }
    __syncthreads();
    int J = misc->ib[2];
    nf = J >= 0 ? J + 1 : nk;
    uint64_t kc = cand[nf - 1];
    vstar = desc_key_val(kc);
    istar = (int32_t)desc_key_id(kc);
  }
  // final probabilities over positions [0, nf) (sampler.py:76)
  double es2 = 0.0;
#pragma unroll
  for (int q = 0; q < CAP / NT; ++q)
    if (p0 + q < nf) es2 += (double)e[q];
  const double Z2 = block_sum(es2, &misc->red);
  uint64_t k2[CAP / NT];
#pragma unroll
  for (int q = 0; q < CAP / NT; ++q) {
    int pos = p0 + q;
    k2[q] = ~0ull;
    if (pos < nf) {
      float pv = (float)((double)e[q] / Z2);
      k2[q] = ((uint64_t)desc_key_id(cand[pos]) << 32) | __float_as_uint(pv);
    }
  }
  const int P2 = next_pow2(nf < 2 ? 2 : nf);
  __syncthreads();
#pragma unroll
  for (int q = 0; q < CAP / NT; ++q) {
    int pos = p0 + q;
    if (pos < P2) cand[pos] = k2[q];
  }
  __syncthreads();
  lds_bitonic_sort(cand, P2);

  // inverse CDF in token-id order
  const double ud = (double)u;
  float pp[CAP / NT];
  double ps = 0.0;
  int64_t lastpos = -1;
#pragma unroll
  for (int q = 0; q < CAP / NT; ++q) {
    int pos = p0 + q;
    pp[q] = pos < nf ? __uint_as_float((uint32_t)cand[pos]) : 0.0f;
    ps += (double)pp[q];
    if (pos < nf && pp[q] > 0.0f) lastpos = pos;
  }
  double tot2;
  double run2 = block_excl_scan(ps, &tot2, &misc->red);
#pragma unroll
  for (int q = 0; q < CAP / NT; ++q) {
    int pos = p0 + q;
    if (pos < nf) {
      double before = run2;
      run2 += (double)pp[q];
      if (run2 > ud && !(before > ud)) misc->ib[3] = pos;
    }
  }
  lastpos = block_max_i64(lastpos, &misc->red);  // barriers order the ib[3] writes
  int pick = misc->ib[3];
  if (pick < 0) pick = lastpos >= 0 ? (int)lastpos : 0;
  const int64_t token = (int64_t)(cand[pick] >> 32);
  if (tid == 0) put_id(o.out_ids, o.row, token);
  write_info(o, path, nf, thr, n_topk, n, flags, vstar, istar);
  if (o.out_probs != nullptr) {
    zero_probs(o);
    float* pr = o.out_probs + (int64_t)o.row * o.V;
    for (int i = tid; i < nf; i += NT) pr[cand[i] >> 32] = __uint_as_float((uint32_t)cand[i]);
  }
}

// State handed from the kernel to the generic (histogram) path.
struct GCtx {
  const uint4* rowv;
  uint32_t* bm;
  float* xl_val;
  int32_t* xl_id;
  uint64_t* cand;
  uint32_t* hcnt;
  uint64_t* hmass;
  Misc* misc;
  IdSink out_ids;
  float* out_probs;
  int32_t* out_info;
  int64_t V, nch, nrows_j;
  int row, U, k, flags;
  float pen, rpen, tdiv, rdiv, p32, Mx, My, u;   // rpen: RN(1/p), read only when recip
  bool pen_on, topk_on, topp_on, recip;
};

// Rows not resolved by the greedy, NaN-guard or small-k paths: top-k for
// large k (count histogram), top-p over large sets (fixed-point mass
// histogram), and the inverse-CDF draw over a large kept set.  Every pass
// re-reads the row (served from L2 / Infinity Cache after P1).
template <typename T>
__device__ __attribute__((always_inline)) inline void generic_path(const GCtx g) {
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wid = wave_id();
  const bool rowthr = tid < RT;
  const bool hwave = wid == NWAVE - 1;
  constexpr int EPC = T::EPC;
  const uint4* rowv = g.rowv;
  const uint32_t* bm = g.bm;
  const float* xl_val = g.xl_val;
  const int32_t* xl_id = g.xl_id;
  uint64_t* cand = g.cand;
  uint32_t* hcnt = g.hcnt;
  uint64_t* hmass = g.hmass;
  Misc* misc = g.misc;
  BlockScratch* red = &misc->red;
  const int64_t V = g.V, nch = g.nch, nrows_j = g.nrows_j;
  const int row = g.row, U = g.U, k = g.k;
  int32_t flags = g.flags;
  const float pen = g.pen, tdiv = g.tdiv, rdiv = g.rdiv, p32 = g.p32, Mx = g.Mx, My = g.My, u = g.u;
  const bool pen_on = g.pen_on, topk_on = g.topk_on, topp_on = g.topp_on;
  const RowOut o{g.out_ids, g.out_probs, g.out_info, row, V};
  struct { IdSink out_ids; float* out_probs; } P{g.out_ids, g.out_probs};

  // ================= generic path: histogram passes over re-read data =================
  // Extras (history wave) contribute through `xl_each`.
  auto xl_each = [&](auto&& f) {
    if (hwave)
      for (int i = lane; i < U; i += 64) f(xl_val[i], (int64_t)xl_id[i]);
  };
  auto row_each = [&](auto&& f) {
    if (rowthr) visit_rows<T>(rowv, bm, pen_on, nch, nrows_j, [&](float x, int64_t id, int64_t) { f(x, id); });
  };
  auto compact = [&](auto&& pred) -> int {
    if (tid == 0) misc->cand_n = 0;
    __syncthreads();
    if (rowthr) {
      for (int64_t j = 0; j < nrows_j; ++j) {
        const int64_t c = j * RT + tid;
        const bool ok = c < nch;
        uint4 w = ok ? rowv[c] : ninf_chunk<T>();
        if (ok && pen_on) w = T::mask(w, T::bits(bm, c));
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          const float x = T::elem(w, e);
          cand_append(ok && pred(x, c * EPC + e), x, c * EPC + e, cand, misc);
        }
      }
    } else {
      for (int base = 0; base < U; base += 64) {
        const int i = base + lane;
        const float x = i < U ? xl_val[i] : NEG_INF;
        const int64_t id = i < U ? xl_id[i] : 0;
        cand_append(i < U && pred(x, id), x, id, cand, misc);
      }
    }
    __syncthreads();
    return misc->cand_n;
  };

  // ---- top-k for large k (or candidate overflow): count histogram in x
  float Lx = NEG_INF;
  float thr_y = NEG_INF;
  int32_t n_topk = (int32_t)V;
  if (topk_on) {
    float lmin = POS_INF;
    int cntf = 0;
    auto f_min = [&](float x, int64_t) { if (x > NEG_INF) { lmin = __builtin_fminf(lmin, x); ++cntf; } };
    row_each(f_min);
    xl_each(f_min);
    const float lo0 = block_min_nan(lmin, red);
    const int64_t nfinite = block_sum_i64(cntf, red);
    float thr_x = NEG_INF;
    if (nfinite >= k) {
      Levels L;
      L.n = 0;
      double hi = Mx, lo = lo0;
      int kk = k;
      bool done = false;
      for (int r = 0; r < MAX_LEVELS && !done; ++r) {
        if (!(hi > lo)) { thr_x = (float)hi; done = true; break; }
        const double s = (double)NB / (hi - lo);
        for (int i = tid; i < NB; i += NT) hcnt[i] = 0u;
        __syncthreads();
        auto f_h = [&](float x, int64_t) {
          if (x > NEG_INF && L.member(x)) atomicAdd(&hcnt[Levels::bin(hi, s, x)], 1u);
        };
        row_each(f_h);
        xl_each(f_h);
        __syncthreads();
        double before;
        const int b = find_bin(nullptr, hcnt, false, (double)kk, false, &before, misc);
        const int cntb = (int)hcnt[b < 0 ? 0 : b];
        __syncthreads();
        if (b < 0) { flags |= FLAG_REFINE_LIMIT; thr_x = (float)lo; done = true; break; }
        kk -= (int)before;
        L.set(r, hi, s, b);
        if (cntb <= CAP || r == MAX_LEVELS - 1) {
          if (cntb > CAP) flags |= FLAG_REFINE_LIMIT;
          const int n = compact([&](float x, int64_t) { return x > NEG_INF && L.member(x); });
          const int nn = n < CAP ? n : CAP;
          // sort the bin's members descending and take the kk-th
          uint64_t kv[CAP / NT];
#pragma unroll
          for (int q = 0; q < CAP / NT; ++q) {
            const int i = tid + q * NT;
            kv[q] = i < nn ? desc_key(__uint_as_float((uint32_t)(cand[i] >> 32)), (uint32_t)cand[i]) : ~0ull;
          }
          const int P2 = next_pow2(nn < 2 ? 2 : nn);
          __syncthreads();
#pragma unroll
          for (int q = 0; q < CAP / NT; ++q) {
            const int i = tid + q * NT;
            if (i < P2) cand[i] = kv[q];
          }
          __syncthreads();
          lds_bitonic_sort(cand, P2);
          const int pos = kk - 1 < nn - 1 ? kk - 1 : nn - 1;
          thr_x = desc_key_val(cand[pos < 0 ? 0 : pos]);
          __syncthreads();
          done = true;
          break;
        }
        const double h0v = hi;
        hi = h0v - (double)b / s;
        lo = h0v - (double)(b + 1) / s;
      }
    }
    Lx = lower_preimage(thr_x, tdiv, rdiv);
    thr_y = div_rn(thr_x, tdiv, rdiv);
    int cnt = 0;
    auto f_c = [&](float x, int64_t) { if (x >= Lx && x > NEG_INF) ++cnt; };
    row_each(f_c);
    xl_each(f_c);
    n_topk = (int32_t)block_sum_i64(cnt, red);
    if (n_topk <= CAP) {
      const int n = compact([&](float x, int64_t) { return x >= Lx; });
      lds_set(n, true, k, topp_on, p32, My, tdiv, rdiv, u, cand, misc, o, PATH_GENERIC_SET, flags, NEG_INF, 0);
      return;
    }
  }

  // ---- top-p on a large set: fixed-point mass histogram in y = x / t
  bool cut = false;
  float vstar = NEG_INF;
  int64_t istar = -1;
  int64_t n_kept = -1;
  if (topp_on) {
    Levels L;
    L.n = 0;
    double hi = My, lo = (double)My - 64.0;
    double above_fx = 0.0;     // fixed-point mass of elements ranked above the current level's bins
    int64_t above_cnt = 0;
    double Zfx = 0.0;
    bool done = false;
    for (int r = 0; r < MAX_LEVELS && !done; ++r) {
      const double s = (double)NB / (hi - lo);
      for (int i = tid; i < NB; i += NT) { hcnt[i] = 0u; hmass[i] = 0ull; }
      __syncthreads();
      auto f_h = [&](float x, int64_t) {
        if (x >= Lx) {
          const float y = div_rn(x, tdiv, rdiv);
          if (y >= (float)((double)My - 64.0) && L.member(y)) {
            const int b = Levels::bin(hi, s, y);
            atomicAdd(&hcnt[b], 1u);
            atomicAdd((unsigned long long*)&hmass[b], (unsigned long long)mass_fx(ns_expf(y - My)));
          }
        }
      };
      row_each(f_h);
      xl_each(f_h);
      __syncthreads();
      if (r == 0) {
        int64_t zz = (int64_t)(hmass[2 * tid] + hmass[2 * tid + 1]);
        Zfx = (double)block_sum_i64(zz, red);
      }
      const double target = (double)p32 * Zfx - above_fx;
      double before;
      const int b = find_bin(hmass, nullptr, true, target, true, &before, misc);
      if (b < 0) { done = true; cut = false; break; }  // the nucleus holds everything
      // count of elements in bins before b
      int c0 = (2 * tid < b ? (int)hcnt[2 * tid] : 0) + (2 * tid + 1 < b ? (int)hcnt[2 * tid + 1] : 0);
      const int64_t cnt_before = block_sum_i64(c0, red);
      const int cntb = (int)hcnt[b];
      __syncthreads();
      L.set(r, hi, s, b);
      above_fx += before;
      above_cnt += cnt_before;
      if (cntb <= CAP || r == MAX_LEVELS - 1) {
        if (cntb > CAP) flags |= FLAG_REFINE_LIMIT;
        const int n = compact([&](float x, int64_t) {
          if (!(x >= Lx)) return false;
          const float y = div_rn(x, tdiv, rdiv);
          return y >= (float)((double)My - 64.0) && L.member(y);
        });
        const int nn = n < CAP ? n : CAP;
        uint64_t kv[CAP / NT];
#pragma unroll
        for (int q = 0; q < CAP / NT; ++q) {
          const int i = tid + q * NT;
          kv[q] = ~0ull;
          if (i < nn) {
            const float y = div_rn(__uint_as_float((uint32_t)(cand[i] >> 32)), tdiv, rdiv);
            kv[q] = desc_key(y, (uint32_t)cand[i]);
          }
        }
        const int P2 = next_pow2(nn < 2 ? 2 : nn);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < CAP / NT; ++q) {
          const int i = tid + q * NT;
          if (i < P2) cand[i] = kv[q];
        }
        if (tid == 0) misc->ib[2] = -1;
        __syncthreads();
        lds_bitonic_sort(cand, P2);
        // exact crossing inside the bin: c_j = fl32(base + sum of fl32(e/Z))
        const double Z = Zfx * FX_INV;
        const double base_q = above_fx / Zfx;
        const int p0 = tid * (CAP / NT);
        float qv[CAP / NT];
        double qs = 0.0;
#pragma unroll
        for (int q = 0; q < CAP / NT; ++q) {
          const int pos = p0 + q;
          qv[q] = pos < nn ? (float)((double)ns_expf(desc_key_val(cand[pos]) - My) / Z) : 0.0f;
          qs += (double)qv[q];
        }
        double tot;
        double run = base_q + block_excl_scan(qs, &tot, red);
#pragma unroll
        for (int q = 0; q < CAP / NT; ++q) {
          const int pos = p0 + q;
          if (pos < nn) {
            const float cprev = (float)run;
            run += (double)qv[q];
            if ((float)run > p32 && (pos == 0 ? !((float)base_q > p32) : !(cprev > p32))) misc->ib[2] = pos;
          }
        }
        __syncthreads();
        int J = misc->ib[2];
        if (J < 0) J = nn - 1;
        const uint64_t kc = cand[J];
        vstar = desc_key_val(kc);
        istar = (int64_t)desc_key_id(kc);
        cut = true;
        n_kept = above_cnt + J + 1;
        __syncthreads();
        done = true;
        break;
      }
      const double h0v = hi;
      hi = h0v - (double)b / s;
      lo = h0v - (double)(b + 1) / s;
    }
  }
  auto keep = [&](float x, int64_t id) -> bool {
    if (!(x >= Lx) || !(x > NEG_INF)) return false;
    if (!cut) return true;
    const float y = div_rn(x, tdiv, rdiv);
    return y > vstar || (y == vstar && id <= istar);
  };
  if (n_kept < 0) {
    int cnt = 0;
    auto f_c = [&](float x, int64_t id) { if (keep(x, id)) ++cnt; };
    row_each(f_c);
    xl_each(f_c);
    n_kept = block_sum_i64(cnt, red);
  }
  if (n_kept <= CAP) {
    const int n = compact(keep);
    lds_set(n, false, k, false, p32, My, tdiv, rdiv, u, cand, misc, o, PATH_GENERIC_SET, flags, thr_y, n_topk);
    return;
  }

  // ---- large kept set: inverse CDF over per-chunk-row mass sums
  {
    // LDS: rowsum[(nrows_j + 1) * NWAVE] doubles and xrow[nrows_j + 1] fixed-point, in the histogram area
    double* rowsum = reinterpret_cast<double*>(hmass);
    uint64_t* xrow = reinterpret_cast<uint64_t*>(cand);
    const int64_t nrow_tot = nrows_j + 1;   // last row = tail elements
    for (int64_t i = tid; i < nrow_tot * NWAVE; i += NT) rowsum[i] = 0.0;
    for (int64_t i = tid; i < nrow_tot; i += NT) xrow[i] = 0ull;
    __syncthreads();
    int64_t lastid = -1;
    double zsum = 0.0;
    if (rowthr) {
      for (int64_t j = 0; j < nrows_j; ++j) {
        const int64_t c = j * RT + tid;
        const bool ok = c < nch;
        uint4 w = ok ? rowv[c] : ninf_chunk<T>();
        if (ok && pen_on) w = T::mask(w, T::bits(bm, c));
        double s = 0.0;
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          const float x = T::elem(w, e);
          if (ok && keep(x, c * EPC + e)) {
            const float ev = ns_expf(div_rn(x, tdiv, rdiv) - My);
            s += (double)ev;
            if (ev > 0.0f) lastid = c * EPC + e;
          }
        }
        zsum += s;
        s = wave_sum(s);
        if (lane == 0) rowsum[j * NWAVE + wid] = s;
      }
    } else {
      for (int i = lane; i < U; i += 64) {
        const float x = xl_val[i];
        const int64_t id = xl_id[i];
        if (keep(x, id)) {
          const float ev = ns_expf(div_rn(x, tdiv, rdiv) - My);
          const int64_t rj = id < nch * EPC ? (id / EPC) / RT : nrows_j;
          atomicAdd((unsigned long long*)&xrow[rj], (unsigned long long)mass_fx(ev));
          if (ev > 0.0f && id > lastid) lastid = id;
        }
      }
    }
    lastid = block_max_i64(lastid, red);
    // row totals and the row holding the crossing (wave 0, two rows per lane)
    if (wid == 0) {
      double tsum[2] = {0.0, 0.0};
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int64_t rj = lane * 2 + q;
        if (rj < nrow_tot) {
          double t = (double)xrow[rj] * FX_INV;
          for (int w = 0; w < NWAVE; ++w) t += rowsum[rj * NWAVE + w];
          tsum[q] = t;
        }
      }
      const double pair = tsum[0] + tsum[1];
      const double incl = wave_incl_scan(pair);
      const double Z = __shfl(incl, 63);
      const double Tu = (double)u * Z;
      const double excl = incl - pair;
      int found = -1;
      double bef = 0.0;
      if (excl <= Tu && excl + tsum[0] > Tu) { found = lane * 2; bef = excl; }
      else if (excl + tsum[0] <= Tu && excl + pair > Tu) { found = lane * 2 + 1; bef = excl + tsum[0]; }
      const uint64_t fm = ballot(found >= 0 && found < nrow_tot);
      if (lane == 0) { misc->ib[5] = -1; misc->db[0] = Tu; misc->db[1] = Z; }
      if (fm != 0ull) {
        const int fl = __builtin_ctzll(fm);
        if (lane == fl) { misc->ib[5] = found; misc->db[2] = bef; }
      }
    }
    __syncthreads();
    const int jstar = misc->ib[5];
    const double Tt = misc->db[0] - misc->db[2];
    int64_t token = -1;
    if (jstar < 0) {
      token = lastid;
    } else if (jstar == nrows_j) {
      // tail row: extras with ids beyond the chunk layout, in id order (at most EPC-1 of them)
      if (tid == 0) {
        double run = 0.0;
        int64_t last = -1;
        for (int64_t id = nch * EPC; id < V && token < 0; ++id) {
          for (int i = 0; i < U; ++i) {
            if (xl_id[i] == id && keep(xl_val[i], id)) {
              const float ev = ns_expf(div_rn(xl_val[i], tdiv, rdiv) - My);
              run += (double)ev;
              if (ev > 0.0f) last = id;
              if (run > Tt) token = id;
            }
          }
        }
        misc->ib[6] = (int)(token >= 0 ? token : (last >= 0 ? last : lastid));
      }
      __syncthreads();
      token = misc->ib[6];
    } else {
      // chunk row jstar: per-thread chunk masses (history positions recomputed), scan, walk
      const int64_t c = (int64_t)jstar * RT + tid;
      const bool ok = rowthr && c < nch;
      float xe[EPC];
      double mt = 0.0;
      uint4 w = ok ? rowv[c] : ninf_chunk<T>();
      const uint32_t hb = (ok && pen_on) ? T::bits(bm, c) : 0u;
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        float x = T::elem(w, e);
        if ((hb >> e) & 1u) x = penalize(x, pen, g.rpen, g.recip);
        float ev = 0.0f;
        if (ok && keep(x, c * EPC + e)) ev = ns_expf(div_rn(x, tdiv, rdiv) - My);
        xe[e] = ev;
        mt += (double)ev;
      }
      double tot;
      const double pre = block_excl_scan(mt, &tot, red);
      if (tid == 0) { misc->ib[6] = -1; misc->ib[7] = -1; }
      __syncthreads();
      if (ok && mt > 0.0) {
        double run = pre;
        int64_t lastk = -1;
        for (int e = 0; e < EPC; ++e) {
          if (xe[e] > 0.0f) {
            const double b4 = run;
            run += (double)xe[e];
            lastk = c * EPC + e;
            if (run > Tt && !(b4 > Tt)) misc->ib[6] = (int)(c * EPC + e);
          }
        }
        atomicMax(&misc->ib[7], (int)lastk);
      }
      __syncthreads();
      token = misc->ib[6];
      if (token < 0) {
        flags |= FLAG_LOCATE_FALLBACK;
        token = misc->ib[7] >= 0 ? misc->ib[7] : lastid;
      }
    }
    if (tid == 0) put_id(P.out_ids, row, token < 0 ? 0 : token);
    write_info(o, PATH_LARGE_DRAW, (int32_t)n_kept, thr_y, n_topk, -1, flags, vstar, (int32_t)istar);
    if (P.out_probs != nullptr) {
      const double Z = misc->db[1];
      __syncthreads();
      float* pr = P.out_probs + (int64_t)row * V;
      if (rowthr) {
        for (int64_t cc = tid; cc < nch; cc += RT) {
          uint4 w2 = rowv[cc];
          if (pen_on) w2 = T::mask(w2, T::bits(bm, cc));
#pragma unroll
          for (int e = 0; e < EPC; ++e) {
            const float x = T::elem(w2, e);
            const int64_t id = cc * EPC + e;
            pr[id] = keep(x, id) ? (float)((double)ns_expf(div_rn(x, tdiv, rdiv) - My) / Z) : 0.0f;
          }
        }
      } else {
        for (int64_t id = nch * EPC + lane; id < V; id += 64) pr[id] = 0.0f;
      }
      __syncthreads();
      if (hwave)
        for (int i = lane; i < U; i += 64) {
          const float x = xl_val[i];
          const int64_t id = xl_id[i];
          pr[id] = keep(x, id) ? (float)((double)ns_expf(div_rn(x, tdiv, rdiv) - My) / Z) : 0.0f;
        }
    }
  }
}

}  // namespace ns

#include "ns_topk.h"

namespace ns {

// Every row kind: P1 streaming with group maxima, the small-k LDS set path and the
// histogram paths.  Called for rows the streaming path does not take.  Inlined (as is
// everything it calls): a call would give the kernel a private segment for the callee's
// saved registers, and a kernel with any private segment dispatches measurably slower
// even when no wave touches it.  The kernel's argument block is read in place.
typedef const KParams* KArgs;

template <typename T>
__device__ __attribute__((always_inline, cold)) inline void row_general(KArgs PA, const int row) {
  const KParams P = *PA;
  extern __shared__ __align__(16) unsigned char smem[];
  Misc* misc = reinterpret_cast<Misc*>(smem);
  uint32_t* bm = reinterpret_cast<uint32_t*>(smem + P.off_bm);
  uint64_t* cand = reinterpret_cast<uint64_t*>(smem + P.off_cand);
  uint32_t* hcnt = reinterpret_cast<uint32_t*>(smem + P.off_hist);
  uint64_t* hmass = reinterpret_cast<uint64_t*>(smem + P.off_hist + 4u * NB);
  BlockScratch* red = &misc->red;

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wid = wave_id();
  const bool rowthr = tid < RT;
  const bool hwave = wid == NWAVE - 1;
  const int64_t V = P.vocab;
  constexpr int EPC = T::EPC;
  const int64_t nch = V / EPC;
  const int ntail = (int)(V - nch * EPC);
  const int64_t nrows_j = (nch + RT - 1) / RT;
  const RowOut o{P.out_ids, P.out_probs, P.out_info, row, V};

  // ---- row parameters (uniform across the workgroup)
  const int64_t src = P.sample_idx ? P.sample_idx[row] : (int64_t)row;
  const float temp = P.temperature[row];
  const float topp = P.top_p[row];
  const float pen = P.penalty[row];
  const float rpen_g = P.pen_rcp != nullptr ? P.pen_rcp[row] : 0.0f;   // the reciprocal penalty's RN(1/p)
  float u = P.uniforms[row];
  u = (u >= 0.0f) ? (u < 1.0f ? u : 0x1.fffffep-1f) : 0.0f;
  const int32_t k = P.top_k[row];
  int32_t h0 = 0, h1 = 0;
  row_history(P.hist_off, P.hist_slot, P.hist_len, P.hist_nslots, P.hist_cap, row, h0, h1);
  const int32_t H = h1 - h0;
  const bool pen_on = (pen != 1.0f) && H > 0;                            // sampler.py:33
  // the extras list (unique history ids, then the tail) in LDS, or for a history with
  // more distinct ids than LDS holds, in the row's region of the workspace
  const int64_t umax = pen_on ? (H < V ? H : V) : 0;
  const bool xl_lds = umax <= P.xcap - 8;
  int32_t flags = 0;
  if (src < 0 || src >= P.n_rows_total) flags |= FLAG_BAD_ROW;
  if (h1 < h0 || H > MAX_HIST || (!xl_lds && (P.xl_glob == nullptr || umax > P.xg_cap - 8)))
    flags |= FLAG_HIST_TOO_LONG;
  if (flags != 0) {
    if (tid == 0) put_id(P.out_ids, row, -1);
    write_info(o, PATH_ERROR, 0, 0.0f, 0, 0, flags, 0.0f, -1);
    return;
  }
  float* xl_val;
  int32_t* xl_id;
  if (xl_lds) {
    xl_val = reinterpret_cast<float*>(smem + P.off_xl);
    xl_id = reinterpret_cast<int32_t*>(smem + P.off_xl + 4u * (uint32_t)P.xcap);
  } else {
    xl_val = P.xl_glob + (int64_t)row * 2 * P.xg_cap;
    xl_id = reinterpret_cast<int32_t*>(xl_val + P.xg_cap);
  }
  const unsigned char* rowp = (const unsigned char*)P.logits + src * P.row_stride * T::SZ;
  const uint4* rowv = reinterpret_cast<const uint4*>(rowp);
  const bool greedy = temp == 0.0f;
  const float tdiv = temp > 0.0f ? __builtin_fmaxf(temp, 1e-6f) : 1.0f;  // sampler.py:42
  const float rdiv = 1.0f / tdiv;
  const bool topk_on = k > 0 && (int64_t)k < V;                          // sampler.py:55
  const bool topp_on = topp < 1.0f;                                      // sampler.py:63
  const float p32 = topp;


  // ---- phase 0: history ids (all threads), then the row loads, zero LDS state
  int32_t hid[HPT];
  {
    const int32_t* hp = P.hist_ids + h0;
#pragma unroll
    for (int s = 0; s < HPT; ++s) {
      const int32_t i = s * NT + tid;
      hid[s] = -1;
      if (pen_on && i < H) hid[s] = hp[i];
    }
  }
  if (pen_on) {
    const int nbw = (int)((V + 31) / 32);
    for (int i = tid; i < nbw; i += NT) bm[i] = 0u;
  }
  if (tid == 0) { misc->xl_n = 0; misc->cand_n = 0; misc->flags = 0; }
  __syncthreads();

  // ---- phase 1: presence bitmap and unique history ids (set semantics, sampler.py:34-38);
  // the first 8192 ids from registers, any further ones streamed in batches of NT
  if (pen_on) {
    auto mark = [&](int32_t id, bool act) {   // every lane of the wave calls it
      const bool valid = act && id >= 0 && (int64_t)id < V;
      if (act && !valid) atomicOr(&misc->flags, FLAG_BAD_HIST_ID);
      bool uniq = false;
      if (valid) {
        const uint32_t bit = 1u << (id & 31);
        const uint32_t old = atomicOr(&bm[id >> 5], bit);
        uniq = (old & bit) == 0u;
      }
      const uint64_t m = ballot(uniq);
      if (m != 0ull) {
        int base = 0;
        if (lane == 0) base = atomicAdd(&misc->xl_n, __popcll(m));
        base = __shfl(base, 0);
        if (uniq) xl_id[base + lanes_below(m)] = id;
      }
    };
#pragma unroll
    for (int s = 0; s < HPT; ++s)
      if (s * NT < H) mark(hid[s], s * NT + tid < H);
    const int32_t* hp = P.hist_ids + h0;
    for (int32_t b = HPT * NT; b < H; b += NT) {
      const bool act = b + tid < H;
      mark(act ? hp[b + tid] : -1, act);
    }
  }
  __syncthreads();

  // ---- phase 2: history wave gathers and penalizes; row threads run P1
  float tmax = NEG_INF;
  int targ = -1;
  float gm[NGROUP];
#pragma unroll
  for (int g = 0; g < NGROUP; ++g) gm[g] = NEG_INF;
  if (hwave) {
    int U = misc->xl_n;
    if (pen_on) {
      for (int base = 0; base < U; base += 64 * GATHER) {
        float xv[GATHER];
#pragma unroll
        for (int s = 0; s < GATHER; ++s) {
          int i = base + s * 64 + lane;
          xv[s] = i < U ? T::load1(rowp, xl_id[i]) : 0.0f;
        }
#pragma unroll
        for (int s = 0; s < GATHER; ++s) {
          int i = base + s * 64 + lane;
          if (i < U) xl_val[i] = penalize(xv[s], pen, rpen_g, P.pen_rcp != nullptr);
        }
      }
    }
    if (ntail > 0) {
      const bool act = lane < ntail;
      const int64_t id = nch * EPC + lane;
      const bool inhist = act && pen_on && ((bm[id >> 5] >> (id & 31)) & 1u);
      const bool take = act && !inhist;
      const float x = take ? T::load1(rowp, id) : 0.0f;
      const uint64_t m = ballot(take);
      const int pos = U + lanes_below(m);
      if (take) { xl_id[pos] = (int32_t)id; xl_val[pos] = x; }
      U += __popcll(m);
    }
    if (lane == 0) misc->xl_n = U;
  } else {
    const int64_t jg = (nrows_j + NGROUP - 1) / NGROUP;
#pragma unroll
    for (int g = 0; g < NGROUP; ++g) {
      const int64_t j0 = g * jg;
      const int64_t j1 = j0 + jg < nrows_j ? j0 + jg : nrows_j;
      float gmax = NEG_INF;
      for (int64_t j = j0; j < j1; j += 4) {
        uint4 v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t c = (j + q) * RT + tid;
          v[q] = (j + q < j1 && c < nch) ? rowv[c] : ninf_chunk<T>();
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t c = (j + q) * RT + tid;
          if (j + q < j1 && c < nch) {
            if (pen_on) v[q] = T::mask(v[q], T::bits(bm, c));
            const float m = chunk_max<T>(v[q]);
            if (m > tmax || (m != m && tmax == tmax)) { tmax = m; targ = (int)(j + q); }
            gmax = fmax_nan(gmax, m);
          }
        }
      }
      gm[g] = gmax;
    }
  }
  __syncthreads();
  const int U = misc->xl_n;
  flags |= misc->flags;
  // small-k rows: the bound from the exact group maxima, which are then kept only
  // rounded up to bfloat16, two per register, for the candidate pass (a larger value
  // merely rescans a group)
  const bool small_topk = !greedy && topk_on && k <= KSMALL;
  const float tau = small_topk ? select_tau<NGROUP>(gm, rowthr, k, hcnt, misc) : NEG_INF;
  uint32_t gm2[NGROUP / 2];
#pragma unroll
  for (int g = 0; g < NGROUP; ++g) {
    const uint32_t gb = __float_as_uint(gm[g]);
    const uint32_t up = (gb >> 31) == 0u && (gb & 0xffffu) != 0u ? (gb >> 16) + 1u : gb >> 16;
    if (g & 1) gm2[g >> 1] |= up << 16;
    else gm2[g >> 1] = up;
  }

  // ---- row max over chunks and extras
  float my = rowthr ? tmax : NEG_INF;
  if (hwave)
    for (int i = lane; i < U; i += 64) my = fmax_nan(my, xl_val[i]);
  const float Mx = block_max_nan(my, red);
  const float My = div_rn(Mx, tdiv, rdiv);

  // ---- greedy rows: first index of the maximum (sampler.py:82-83, 88)
  if (greedy) {
    const bool nanrow = Mx != Mx;
    int64_t best = INT64_MAX;
    if (rowthr) {
      {
        if (nanrow) {
          visit_rows<T>(rowv, bm, pen_on, nch, nrows_j, [&](float x, int64_t id, int64_t) {
            if (x != x && id < best) best = id;
          });
        } else if (targ >= 0 && tmax == Mx) {
          const int64_t c = (int64_t)targ * RT + tid;
          uint4 w = rowv[c];
          if (pen_on) w = T::mask(w, T::bits(bm, c));
#pragma unroll
          for (int e = 0; e < EPC; ++e)
            if (T::elem(w, e) == Mx && c * EPC + e < best) best = c * EPC + e;
        }
      }
    }
    if (hwave)
      for (int i = lane; i < U; i += 64) {
        const float x = xl_val[i];
        if ((nanrow ? (x != x) : (x == Mx)) && xl_id[i] < best) best = xl_id[i];
      }
    best = block_min_i64(best, red);
    if (tid == 0) put_id(P.out_ids, row, best == INT64_MAX ? 0 : best);
    write_info(o, PATH_GREEDY, 1, NEG_INF, 0, 0, flags, Mx, (int32_t)best);
    return;
  }

  // ---- rows whose softmax is NaN: uniform 1/V over the vocabulary (sampler.py:77-80)
  if (!(__builtin_fabsf(My) <= FLT_MAXV)) {
    const float q = uniform_q(V);
    if (tid == 0) put_id(P.out_ids, row, uniform_pick(u, q, V));
    write_info(o, PATH_UNIFORM, (int32_t)V, NEG_INF, (int32_t)V, 0, flags, My, -1);
    if (P.out_probs != nullptr) {
      float* pr = P.out_probs + (int64_t)row * V;
      for (int64_t i = tid; i < V; i += NT) pr[i] = q;
    }
    return;
  }

  // ---- top-k with k <= KSMALL: threshold from chunk maxima, candidates to LDS
  if (small_topk) {
    const float tc = lower_preimage(tau, tdiv, rdiv);
    if (tid == 0) misc->cand_n = 0;
    __syncthreads();
    if (hwave) {
      for (int base = 0; base < U; base += 64) {
        const int i = base + lane;
        const float x = i < U ? xl_val[i] : NEG_INF;
        cand_append(i < U && x >= tc, x, i < U ? xl_id[i] : 0, cand, misc);
      }
    } else {
      const int64_t jg = (nrows_j + NGROUP - 1) / NGROUP;
#pragma unroll
      for (int g = 0; g < NGROUP; ++g) {
        const float gmg = __uint_as_float((g & 1) ? (gm2[g >> 1] & 0xffff0000u) : (gm2[g >> 1] << 16));
        if (ballot(gmg >= tc) != 0ull) {
          const bool hitg = gmg >= tc;
          const int64_t j0 = g * jg;
          const int64_t j1 = j0 + jg < nrows_j ? j0 + jg : nrows_j;
          for (int64_t j = j0; j < j1; ++j) {
            const int64_t c = j * RT + tid;
            const bool ok = hitg && c < nch;
            uint4 w = ok ? rowv[c] : ninf_chunk<T>();
            if (ok && pen_on) w = T::mask(w, T::bits(bm, c));
#pragma unroll
            for (int e = 0; e < EPC; ++e) {
              const float x = T::elem(w, e);
              cand_append(ok && x >= tc, x, c * EPC + e, cand, misc);
            }
          }
        }
      }
    }
    __syncthreads();
    const int n = misc->cand_n;
    if (n <= CAP) {
      lds_set(n, true, k, topp_on, p32, My, tdiv, rdiv, u, cand, misc, o, PATH_TOPK_SET, flags, NEG_INF, 0);
      return;
    }
    flags |= FLAG_CAND_OVERFLOW;
  }

  generic_path<T>(GCtx{rowv, bm, xl_val, xl_id, cand, hcnt, hmass, misc, P.out_ids, P.out_probs, P.out_info,
                      V, nch, nrows_j, row, U, k, flags, pen, rpen_g, tdiv, rdiv, p32, Mx, My, u, pen_on, topk_on,
                      topp_on, P.pen_rcp != nullptr});
}

// The per-row code for one row: the streaming path for greedy and small-k rows that fit in
// registers, the general code otherwise.  P is the kernel's first argument (the general code
// reads it through the argument segment).
template <typename T>
__device__ __forceinline__ void sample_row(const KParams P, const int row) {
  // every per-row parameter is requested before any is used: one round trip to memory
  // ahead of the row's stream instead of a chain of dependent ones
  const float temp = P.temperature[row];
  const int32_t k = P.top_k[row];
  const float topp = P.top_p[row];
  const float pen = P.penalty[row];
  float u = P.uniforms[row];
  const int64_t src = P.sample_idx ? P.sample_idx[row] : (int64_t)row;
  int32_t h0 = 0, h1 = 0;
  row_history(P.hist_off, P.hist_slot, P.hist_len, P.hist_nslots, P.hist_cap, row, h0, h1);
  if (P.fast) {
    // greedy and small-k rows that fit in registers: one streaming pass
    if (seg_row(temp, k, P.vocab) && row_fits<T>(P.vocab)) {
      if (src >= 0 && src < P.n_rows_total && h0 >= 0 && h1 >= h0 && h1 - h0 <= MAX_HIST &&
          (pen == 1.0f || (h1 - h0 < P.vocab ? h1 - h0 : P.vocab) <= P.xcap - 8)) {
        extern __shared__ __align__(16) unsigned char smem[];
        Misc* misc = reinterpret_cast<Misc*>(smem);
        uint32_t* bm = reinterpret_cast<uint32_t*>(smem + P.off_bm);
        float* xl_val = reinterpret_cast<float*>(smem + P.off_xl);
        int32_t* xl_id = reinterpret_cast<int32_t*>(smem + P.off_xl + 4u * (uint32_t)P.xcap);
        uint64_t* cand = reinterpret_cast<uint64_t*>(smem + P.off_cand);
        u = (u >= 0.0f) ? (u < 1.0f ? u : 0x1.fffffep-1f) : 0.0f;
        const int st = row_fast<T>(RowArgs{P.logits, P.row_stride, P.vocab, P.hist_ids, P.out_ids, P.out_probs,
                                           P.out_info, P.pen_rcp},
                                   row, src, temp, k, topp, pen, u, h0, h1 - h0, 0, misc, bm, xl_id, xl_val, cand);
        if (__builtin_expect(st == 0, 1)) return;
      }
    }
  }
  row_general<T>((KArgs)__builtin_amdgcn_kernarg_segment_ptr(), row);
}

template <typename T>
__global__ __launch_bounds__(NT) void sample_kernel(const KParams P) {
  const int row = blockIdx.x;
  // rows the segment kernel or the wide path resolved carry status 0 (every other row 1):
  // those workgroups end before anything else is read
  if (P.status != nullptr && P.status[row] == 0) return;
  sample_row<T>(P, row);
}

// The last launch of a call with wide rows, one workgroup per sampled row: a wide row the
// cut pass planned is ordered, cut and drawn (wide_final_row); the rows the earlier launches
// left (status 1), and a planned row the final step hands back, take the per-row code, in
// the same workgroup.  The wide step and the per-row code share the dynamic LDS region.
template <typename T>
__global__ __launch_bounds__(NT) void final_kernel(const KParams P, const WideParams W) {
  const int row = blockIdx.x;
  const int32_t step = W.rows[row].step;
  if (step == WSTEP_CUT || step == WSTEP_FULL) {
    extern __shared__ __align__(16) unsigned char smem[];
    wide_final_row<T>(W, *reinterpret_cast<WideSmemCut*>(smem), row);
    // the final step writes status 1 (by thread 0) for a row it hands back; the word past the
    // wide step's LDS tells every thread, and the per-row code reuses the region only after
    // all have read it
    int32_t* rest = reinterpret_cast<int32_t*>(smem + sizeof(WideSmemCut));
    if (threadIdx.x == 0) *rest = P.status[row];
    __syncthreads();
    const int32_t handed_back = *rest;
    __syncthreads();
    if (handed_back == 0) return;
  } else if (P.status[row] == 0) {
    return;
  }
  sample_row<T>(P, row);
}

// One workgroup per sampled row for calls whose rows are all top-k rows with
// 1 <= k <= KFAST (the host's NS_KIND_SMALL_K hint): the row's loads are issued before the
// per-row parameters return (topk_stream, ns_topk.h).  A row of another kind, or one that
// path hands back, is resolved by the general per-row code: the hint never changes a result.
// Word i of a device array through a vector buffer load at a lane offset the compiler cannot
// prove uniform: the load goes out with the wave's other vector loads, in issue order,
// instead of through the scalar cache.  The value is the same in every lane.
__device__ __forceinline__ uint32_t vload_word(const void* base, int32_t i, uint32_t zero) {
  return __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(base, (uint32_t)(i + 1) * 4u), (int)(zero + (uint32_t)i * 4u),
                                              0, 0);
}

template <typename T, int NPH>
__global__ __launch_bounds__(NT) void topk_kernel(const KParams P) {
  const int row = blockIdx.x;
  NS_STAMP_DECL;
  NS_STAMP(0);
  // Without sample indices or device-resident history slots the row and its history range
  // need no dependent load: the per-row parameters are requested first (vector loads, served
  // in issue order ahead of the row) and the row's first chunks right behind them, before the
  // parameters return.  Rows n_sample <= n_rows_total there (checked on the host).
  const bool early = P.sample_idx == nullptr && P.hist_slot == nullptr;
  float temp, topp, pen, u;
  int32_t k, h0 = 0, h1 = 0;
  uint4 v[TK_CPT];
  int64_t src = row;
  if (early) {
    uint32_t zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    const uint32_t wt = vload_word(P.temperature, row, zero), wk = vload_word(P.top_k, row, zero);
    const uint32_t wp = vload_word(P.top_p, row, zero), wr = vload_word(P.penalty, row, zero);
    const uint32_t wu = vload_word(P.uniforms, row, zero);
    uint32_t w0 = 0u, w1 = 0u;
    if (P.hist_off != nullptr) { w0 = vload_word(P.hist_off, row, zero); w1 = vload_word(P.hist_off, row + 1, zero); }
    __builtin_amdgcn_sched_barrier(0);
    topk_issue_early<T, NPH>(v, (const unsigned char*)P.logits + (int64_t)row * P.row_stride * T::SZ, P.vocab);
    temp = __uint_as_float(__builtin_amdgcn_readfirstlane(wt));
    k = (int32_t)__builtin_amdgcn_readfirstlane(wk);
    topp = __uint_as_float(__builtin_amdgcn_readfirstlane(wp));
    pen = __uint_as_float(__builtin_amdgcn_readfirstlane(wr));
    u = __uint_as_float(__builtin_amdgcn_readfirstlane(wu));
    h0 = (int32_t)__builtin_amdgcn_readfirstlane(w0);
    h1 = (int32_t)__builtin_amdgcn_readfirstlane(w1);
  } else {
    temp = P.temperature[row];
    k = P.top_k[row];
    topp = P.top_p[row];
    pen = P.penalty[row];
    u = P.uniforms[row];
    row_history(P.hist_off, P.hist_slot, P.hist_len, P.hist_nslots, P.hist_cap, row, h0, h1);
    if (P.sample_idx != nullptr) src = P.sample_idx[row];
  }
  const int32_t H = h1 - h0;
  const bool pen_on = pen != 1.0f && H > 0;
  const bool ok = src >= 0 && src < P.n_rows_total && h0 >= 0 && H >= 0 && H <= MAX_HIST && temp != 0.0f &&
                  k >= 1 && k <= KFAST && (int64_t)k < P.vocab && !(pen_on && !(pen > 1.0f && pen <= 3.40282347e38f));
  if (ok) {
    extern __shared__ __align__(16) unsigned char smem[];
    Misc* misc = reinterpret_cast<Misc*>(smem);
    uint32_t* bm = reinterpret_cast<uint32_t*>(smem + P.off_bm);
    uint64_t* cand = reinterpret_cast<uint64_t*>(smem + P.off_cand);
    const unsigned char* rowp = (const unsigned char*)P.logits + src * P.row_stride * T::SZ;
    u = (u >= 0.0f) ? (u < 1.0f ? u : 0x1.fffffep-1f) : 0.0f;
    const int st = topk_stream<T, NPH>(RowArgs{P.logits, P.row_stride, P.vocab, P.hist_ids, P.out_ids, P.out_probs,
                                          P.out_info, P.pen_rcp},
                                  row, rowp, v, early, P.hist_ids + h0, temp, k, topp, pen, u, H, misc, bm, cand);
    if (__builtin_expect(st == 0, 1)) return;
  }
  row_general<T>((KArgs)__builtin_amdgcn_kernarg_segment_ptr(), row);
}

}  // namespace ns

#include "ns_split.h"

namespace ns {

// uniforms[rows ? rows[j] : j] = seeded_uniform(seeds[j], steps[j]) for j < n.
__global__ __launch_bounds__(256) void seeded_uniforms_kernel(const uint64_t* seeds, const int64_t* steps,
                                                               const int32_t* rows, int32_t n, float* uniforms) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= n) return;
  uniforms[rows != nullptr ? rows[j] : j] = seeded_uniform(seeds[j], steps[j]);
}

// Zero n16 16-byte words at p (the no-allocation entry point's scratch, once per device).
__global__ __launch_bounds__(256) void scratch_clear_kernel(uint4* p, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// ---- device-resident histories: slot s holds its length in lens[s] and its ids in
// ids[s * cap .. s * cap + lens[s])

// ids[0..n) become slot `slot`'s history (a request's prompt, engine.py:242-243).
__global__ __launch_bounds__(256) void hist_assign_kernel(int32_t* lens, int32_t* ids, int32_t cap, int32_t slot,
                                                          const int32_t* src, int32_t n) {
  int32_t* dst = ids + (int64_t)slot * cap;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) dst[i] = src[i];
  if (blockIdx.x == 0 && threadIdx.x == 0) lens[slot] = n;
}

// Row r's sampled token joins slot slots[r] (scheduler.py:281-284 appending to
// output_token_ids).  One thread per row; the rows of a call name distinct slots.
// A row that failed (id -1: a sample index outside the logits) appends nothing.
__global__ __launch_bounds__(256) void hist_append_kernel(int32_t* lens, int32_t* ids, int32_t nslots, int32_t cap,
                                                          const int32_t* slots, const int64_t* tok, int32_t n,
                                                          int32_t* overflow) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r >= n) return;
  const int32_t s = slots[r];
  if (s < 0 || s >= nslots) return;
  const int64_t t = tok[r];
  if (t < 0) return;
  const int32_t l = lens[s];
  if (l < 0 || l >= cap) {
    if (overflow != nullptr) atomicAdd(overflow, 1);
    return;
  }
  ids[(int64_t)s * cap + l] = (int32_t)t;
  lens[s] = l + 1;
}

// ---- the penalized, temperature-scaled logits of each row (sampler.py:31-38 then :41-51),
// written whole by one of the routines the sampling kernels compute them with:
//   DBG_STREAM  pen_val then div_rn (the streaming, top-k, split and segment kernels);
//   DBG_WIDE    chunk_y (the wide path: multiply-and-correct, IEEE on a chunk out of range);
//   DBG_GENERAL penalize (IEEE division) then div_rn (the per-row general code).
// One workgroup per row; the history bitmap of the whole row in LDS.  A row whose history
// or sample index is invalid is written as NaN.  Not on any sampling path: it exists so
// that each routine can be compared bit for bit with the float32 tensor expression.
enum { DBG_STREAM = 0, DBG_WIDE = 1, DBG_GENERAL = 2 };

template <typename T>
__global__ __launch_bounds__(1024) void debug_scaled_kernel(KParams p, int32_t formula, float* out, int64_t ld_out) {
  extern __shared__ uint32_t bm[];
  constexpr int EPC = T::EPC;
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t V = p.vocab;
  const int64_t nbw = (V + 31) / 32;
  float* orow = out + (int64_t)row * ld_out;
  const int64_t src = p.sample_idx ? p.sample_idx[row] : (int64_t)row;
  int32_t h0 = 0, h1 = 0;
  row_history(p.hist_off, p.hist_slot, p.hist_len, p.hist_nslots, p.hist_cap, row, h0, h1);
  if (src < 0 || src >= p.n_rows_total || h0 < 0 || h1 < h0) {
    for (int64_t i = tid; i < V; i += 1024) orow[i] = __builtin_nanf("");
    return;
  }
  for (int64_t i = tid; i < nbw; i += 1024) bm[i] = 0u;
  __syncthreads();
  for (int32_t i = h0 + tid; i < h1; i += 1024) {
    const int32_t id = p.hist_ids[i];
    if (id >= 0 && id < V) atomicOr(&bm[id >> 5], 1u << (id & 31));
  }
  __syncthreads();

  const float temp = p.temperature[row];
  const float pen = p.penalty[row];
  WRowCtx c{};
  c.row = row;
  c.V = V;
  c.src = src;
  c.rowp = static_cast<const unsigned char*>(p.logits) + src * p.row_stride * T::SZ;
  c.pen = pen;
  c.recip = p.pen_rcp != nullptr;
  c.rpen = c.recip ? p.pen_rcp[row] : 1.0f / pen;
  c.tdiv = temp > 0.0f ? __builtin_fmaxf(temp, 1e-6f) : 1.0f;   // sampler.py:42
  c.rdiv = 1.0f / c.tdiv;
  c.scale = c.tdiv != 1.0f;
  c.lo_t = div_lo(c.tdiv, c.rdiv);
  c.lo_pen = c.recip ? __builtin_inff() : div_lo(pen, c.rpen);   // as wide_row_ctx
  c.pen_on = pen != 1.0f && h1 > h0;                           // sampler.py:33
  const int64_t nch = (V + EPC - 1) / EPC;
  const int64_t nfull = V / EPC;
  const uint4* rowv = reinterpret_cast<const uint4*>(c.rowp);
  // every lane of a wave takes the same number of steps (chunk_y votes across the wave)
  for (int64_t c0 = 0; c0 < nch; c0 += 1024) {
    const int64_t ch = c0 + tid;
    uint4 w = ch < nfull ? rowv[ch] : seg_ninf<T>();
    w = wide_chunk_fix<T>(c, ch, w);
    const uint32_t hb = (ch < nch && c.pen_on) ? T::bits(bm, ch) : 0u;
    float y[EPC];
    if (formula == DBG_WIDE) {
      chunk_y<T>(c, w, hb, ch * EPC, y);
    } else {
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        float x = T::elem(w, e);
        if ((hb >> e) & 1u)
          x = formula == DBG_GENERAL ? penalize(x, pen, c.rpen, c.recip) : pen_rn(x, pen, c.rpen, c.recip);
        y[e] = div_rn(x, c.tdiv, c.rdiv);
      }
    }
#pragma unroll
    for (int e = 0; e < EPC; ++e)
      if (ch * EPC + e < V) orow[ch * EPC + e] = y[e];
  }
}

}  // namespace ns

// =====================================================================================
// C ABI
// =====================================================================================
namespace {
thread_local std::string g_err;
int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

// Segment geometry: elements per segment and segments per row.
int64_t seg_elems(int32_t dtype) { return (int64_t)ns::SEG_CH * (dtype == NS_DTYPE_BF16 ? 8 : 4); }
int64_t seg_count(int64_t vocab, int32_t dtype) { return (vocab + seg_elems(dtype) - 1) / seg_elems(dtype); }
int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// Split-path geometry for n rows of V tokens: S slices of equal length (to a chunk) per row,
// as many as fill about one workgroup per CU, at most SP_MAXS, and at least NT chunks each
// (every thread holds a chunk, so the bound comes from 128 full 8-lane groups: for k <= 64
// about 90 elements reach it); cpt, a power of two up to TK_CPT, covers the longest slice.  Returns S (1: no split; more than SP_MAXS: the rows
// are too long for the slices).
int split_geometry(int64_t n, int64_t V, int32_t dtype, int n_cu, int32_t& cpt, int32_t& nch_out) {
  const int64_t epc = dtype == NS_DTYPE_BF16 ? 8 : 4;
  const int64_t nch = (V + epc - 1) / epc;
  nch_out = (int32_t)(nch < INT32_MAX ? nch : INT32_MAX);
  int64_t S = n > 0 ? (n_cu + n - 1) / n : 1;
  if (S > ns::SP_MAXS) S = ns::SP_MAXS;
  if (S > nch / ns::NT) S = nch / ns::NT;
  const int64_t longest_cap = (int64_t)ns::NT * ns::TK_CPT;
  if (S < (nch + longest_cap - 1) / longest_cap) S = (nch + longest_cap - 1) / longest_cap;
  if (S < 1) S = 1;
  const int64_t longest = (nch + S - 1) / S;
  cpt = 1;
  while ((int64_t)cpt * ns::NT < longest && cpt < ns::TK_CPT) cpt *= 2;
  return S > ns::SP_MAXS ? ns::SP_MAXS + 1 : (int)S;
}

// Device-resident history state: int32 lengths[n_slots] padded to 256 bytes, then int32
// ids[n_slots][capacity].
int hist_state_check(int32_t n_slots, int32_t capacity) {
  if (n_slots <= 0) return fail(NS_ERR_INVALID, "hist_n_slots must be > 0");
  if (capacity <= 0 || capacity > NS_MAX_HISTORY)
    return fail(NS_ERR_INVALID, "hist_capacity must be in [1, " + std::to_string(NS_MAX_HISTORY) + "]");
  if ((int64_t)n_slots * capacity > INT32_MAX) return fail(NS_ERR_INVALID, "hist_n_slots * hist_capacity > 2^31 - 1");
  return NS_OK;
}
const int32_t* hist_state_ids(const void* state, int32_t n_slots) {
  return reinterpret_cast<const int32_t*>(static_cast<const unsigned char*>(state) + align256((int64_t)n_slots * 4));
}

// The no-allocation entry point's workspace: one array per GPU, resident for the life of the
// process.  Host code never uses its name as an address; the address on each device comes
// from hipGetSymbolAddress, once per device, with that device current.
static __device__ __align__(256) unsigned char scratch[NS_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Per-device facts the sampler needs on every call, read once per device: the LDS limit and
// the CU count, and each one-workgroup-per-row kernel's dynamic-LDS limit raised to the
// device's maximum (a call never needs more than the device allows).
struct DevInfo {
  int max_lds = 0;
  int n_cu = 0;
  bool ready = false;
};
std::mutex g_dev_mu;
DevInfo g_dev[kMaxDevices];

int device_info(int dev, DevInfo& out);

// LDS layout of the one-workgroup-per-row kernels: Misc, the row's history bitmap, the
// extras (unique history ids up to LDS_HIST, then the tail), the candidates, the histogram.
struct LdsLayout {
  uint32_t off_bm, off_xl, off_cand, off_hist, total;
  int32_t xcap;
};
LdsLayout lds_layout(int64_t vocab, int32_t max_hist) {
  const int64_t nbw = (vocab + 31) / 32;
  int64_t uniq = max_hist < vocab ? max_hist : vocab;
  if (uniq > ns::LDS_HIST) uniq = ns::LDS_HIST;
  const int64_t xcap = ((uniq + 8 + 3) / 4) * 4;
  LdsLayout l;
  int64_t off = ((int64_t)sizeof(ns::Misc) + 15) / 16 * 16;
  l.off_bm = (uint32_t)off;
  off += (nbw * 4 + 15) / 16 * 16;
  l.off_xl = (uint32_t)off;
  l.xcap = (int32_t)xcap;
  off += (xcap * 8 + 15) / 16 * 16;
  l.off_cand = (uint32_t)off;
  off += (int64_t)ns::CAP * 8;
  l.off_hist = (uint32_t)off;
  off += (int64_t)ns::NB * 12;
  l.total = (uint32_t)off;
  return l;
}

struct WsLayout {
  int64_t counters, status, stats, cand, wrow, shist, slist, smeta, xlong, total;
  int32_t xg_cap;   // extras per row in the xlong region (0: none)
};
// Workspace layout.  The per-row arrival counters are the only state that outlives a
// call (each call leaves them at zero): they sit at fixed positions at the start, sized
// for NS_SEG_MAX_ROWS rows, so calls of any shape sharing one workspace always find
// zeroed counters.  Everything behind them is rewritten by every call before it is read.
WsLayout ws_layout(int32_t n_sample, int64_t vocab, int32_t dtype, int32_t max_hist) {
  const int64_t n = n_sample < NS_SEG_MAX_ROWS ? n_sample : NS_SEG_MAX_ROWS;
  const int64_t rows = (n + 7) / 8 * 8;
  const int64_t S = seg_count(vocab, dtype);
  WsLayout L;
  L.counters = 0;
  L.status = align256((int64_t)NS_SEG_MAX_ROWS * 4);
  L.stats = L.status + align256(rows * 4);
  L.cand = L.stats + align256(rows * S * (int64_t)sizeof(ns::SegStat));
  // wide path: per-row plans and histograms, for up to NS_WIDE_MAX_ROWS rows
  const int64_t wrows = rows < NS_WIDE_MAX_ROWS ? rows : NS_WIDE_MAX_ROWS;
  L.wrow = L.cand + align256(rows * S * ns::SEG_CAP * 8);
  // each wide row's segment histograms (pass 1 to its planner and cut pass)
  L.shist = L.wrow + align256(wrows * (int64_t)sizeof(ns::WideRow));
  // split path: each slice's ordered keys and its word of flags, for up to SP_MAX_ROWS rows
  const int64_t srows = rows < ns::SP_MAX_ROWS ? rows : ns::SP_MAX_ROWS;
  L.slist = L.shist + align256(wrows * S * ns::WBINS * 8);
  L.smeta = L.slist + align256(srows * ns::SP_MAXS * ns::SP_LIST * 8);
  L.xlong = L.smeta + align256(srows * ns::SP_MAXS * (int64_t)sizeof(ns::SplitMeta));
  // histories longer than the general code's LDS list: each row's unique ids and their
  // penalized values (and the tail) in a region of its own, for every row of the call
  const int64_t uniq = max_hist < vocab ? max_hist : vocab;
  L.xg_cap = max_hist > ns::LDS_HIST ? (int32_t)(((uniq + 8 + 3) / 4) * 4) : 0;
  L.total = L.xlong + align256((int64_t)n_sample * L.xg_cap * 8);
  return L;
}
int device_info(int dev, DevInfo& out) {
  if (dev < 0 || dev >= kMaxDevices) return fail(NS_ERR_INVALID, "device index beyond the device table");
  std::lock_guard<std::mutex> lock(g_dev_mu);
  DevInfo& d = g_dev[dev];
  if (!d.ready) {
    hipError_t e = hipDeviceGetAttribute(&d.max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("hipDeviceGetAttribute: ") + hipGetErrorString(e));
    e = hipDeviceGetAttribute(&d.n_cu, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("hipDeviceGetAttribute: ") + hipGetErrorString(e));
    const void* fns[] = {reinterpret_cast<const void*>(&ns::sample_kernel<ns::BF16>),
                         reinterpret_cast<const void*>(&ns::sample_kernel<ns::F32>),
                         reinterpret_cast<const void*>(&ns::topk_kernel<ns::BF16, 1>),
                         reinterpret_cast<const void*>(&ns::topk_kernel<ns::F32, 1>),
                         reinterpret_cast<const void*>(&ns::topk_kernel<ns::BF16, 2>),
                         reinterpret_cast<const void*>(&ns::topk_kernel<ns::F32, 2>),
                         reinterpret_cast<const void*>(&ns::split_kernel<ns::BF16>),
                         reinterpret_cast<const void*>(&ns::split_kernel<ns::F32>),
                         reinterpret_cast<const void*>(&ns::final_kernel<ns::BF16>),
                         reinterpret_cast<const void*>(&ns::final_kernel<ns::F32>)};
    for (const void* fn : fns) {
      e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, d.max_lds);
      if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
    }
    d.ready = true;
  }
  out = d;
  return NS_OK;
}
// Checks the arguments every entry point that reads an ns_sample_args shares (n_sample > 0)
// and fills p's pointers and sizes; has_hist: the call carries histories.
int sample_params(const ns_sample_args* a, ns::KParams& p, bool& has_hist) {
  if (a->logits == nullptr || a->temperature == nullptr || a->top_k == nullptr || a->top_p == nullptr ||
      a->rep_penalty == nullptr || a->uniforms == nullptr || a->out_ids == nullptr)
    return fail(NS_ERR_INVALID, "a required pointer is NULL");
  if (a->dtype != NS_DTYPE_F32 && a->dtype != NS_DTYPE_BF16) return fail(NS_ERR_INVALID, "dtype must be f32 or bf16");
  if (a->vocab <= 0 || a->vocab > NS_MAX_VOCAB)
    return fail(NS_ERR_INVALID, "vocab must be in [1, " + std::to_string(NS_MAX_VOCAB) + "]");
  if (a->row_stride < a->vocab) return fail(NS_ERR_INVALID, "row_stride < vocab");
  if (a->n_rows_total <= 0) return fail(NS_ERR_INVALID, "n_rows_total <= 0");
  if (a->sample_idx == nullptr && a->n_rows_total < a->n_sample)
    return fail(NS_ERR_INVALID, "n_rows_total < n_sample without sample_idx");
  if (a->hist_offsets != nullptr && a->hist_ids == nullptr) return fail(NS_ERR_INVALID, "hist_ids is NULL");
  // history source: CSR offsets and ids, device-resident request slots, or none
  const bool slots = a->hist_state != nullptr;
  if (slots) {
    if (a->hist_offsets != nullptr || a->hist_ids != nullptr)
      return fail(NS_ERR_INVALID, "hist_state excludes hist_offsets and hist_ids");
    if (a->hist_slot == nullptr) return fail(NS_ERR_INVALID, "hist_slot is NULL");
    const int rs = hist_state_check(a->hist_n_slots, a->hist_capacity);
    if (rs != NS_OK) return rs;
  }
  has_hist = a->hist_offsets != nullptr || slots;
  const int32_t* h_ids = slots ? hist_state_ids(a->hist_state, a->hist_n_slots) : a->hist_ids;
  const int32_t* h_len = slots ? static_cast<const int32_t*>(a->hist_state) : nullptr;
  const int32_t* h_slot = slots ? a->hist_slot : nullptr;
  if (a->max_hist < 0 || a->max_hist > NS_MAX_HISTORY)
    return fail(NS_ERR_INVALID, "max_hist must be in [0, " + std::to_string(NS_MAX_HISTORY) + "]");
  const int esz = a->dtype == NS_DTYPE_F32 ? 4 : 2;
  if (((uintptr_t)a->logits % 16) != 0 || ((a->row_stride * esz) % 16) != 0)
    return fail(NS_ERR_ALIGN, "logits rows must start on 16-byte boundaries (base and row stride)");
  p.logits = a->logits;
  p.row_stride = a->row_stride;
  p.vocab = a->vocab;
  p.n_rows_total = a->n_rows_total;
  p.sample_idx = a->sample_idx;
  p.temperature = a->temperature;
  p.top_k = a->top_k;
  p.top_p = a->top_p;
  p.penalty = a->rep_penalty;
  if (a->penalty_rounding == NS_PENALTY_DIVIDE) {
    p.pen_rcp = nullptr;
  } else if (a->penalty_rounding == NS_PENALTY_RECIPROCAL) {
    if (a->rep_penalty_recip == nullptr)
      return fail(NS_ERR_INVALID, "NS_PENALTY_RECIPROCAL needs rep_penalty_recip");
    p.pen_rcp = a->rep_penalty_recip;
  } else {
    return fail(NS_ERR_INVALID, "penalty_rounding must be NS_PENALTY_DIVIDE or NS_PENALTY_RECIPROCAL");
  }
  p.hist_off = a->hist_offsets;
  p.hist_ids = h_ids;
  p.hist_slot = h_slot;
  p.hist_len = h_len;
  p.hist_nslots = a->hist_n_slots;
  p.hist_cap = a->hist_capacity;
  p.uniforms = a->uniforms;
  p.out_ids = ns::IdSink{a->out_ids, nullptr, nullptr, nullptr, nullptr, 0, 0};
  if (a->hist_append != 0) {
    // the kernel that writes a row's id also appends it to the row's slot
    if (!slots) return fail(NS_ERR_INVALID, "hist_append needs hist_state");
    p.out_ids.slot = a->hist_slot;
    p.out_ids.lens = static_cast<int32_t*>(a->hist_state);
    p.out_ids.ids = const_cast<int32_t*>(h_ids);
    p.out_ids.overflow = a->hist_overflow;
    p.out_ids.cap = a->hist_capacity;
    p.out_ids.nslots = a->hist_n_slots;
  }
  p.out_probs = a->out_probs;
  p.out_info = a->out_info;
  p.n_sample = a->n_sample;
  return NS_OK;
}

}  // namespace

extern "C" {

int ns_abi_version(void) { return NS_ABI_VERSION; }

#ifdef NS_PHASE_STAMPS
// The stamps library only (built with NS_PHASE_STAMPS, never shipped): where the top-k
// streaming kernel stores its phase stamps, NS_STAMPS uint64 per workgroup (NULL: none).
int ns_phase_stamps_set(void* buf) {
  const hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(ns::ns_stamp_buf), &buf, sizeof(buf));
  if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("hipMemcpyToSymbol: ") + hipGetErrorString(e));
  return NS_OK;
}
#endif

int ns_hist_state_bytes(int32_t n_slots, int32_t capacity, uint64_t* bytes) {
  if (bytes == nullptr) return fail(NS_ERR_INVALID, "bytes is NULL");
  const int rc = hist_state_check(n_slots, capacity);
  if (rc != NS_OK) return rc;
  *bytes = (uint64_t)(align256((int64_t)n_slots * 4) + (int64_t)n_slots * capacity * 4);
  return NS_OK;
}

int ns_hist_assign(void* state, int32_t n_slots, int32_t capacity, int32_t slot, const int32_t* ids, int32_t n,
                   hipStream_t stream) {
  if (state == nullptr) return fail(NS_ERR_INVALID, "state is NULL");
  int rc = hist_state_check(n_slots, capacity);
  if (rc != NS_OK) return rc;
  if (slot < 0 || slot >= n_slots) return fail(NS_ERR_INVALID, "slot out of range");
  if (n < 0 || n > capacity) return fail(NS_ERR_INVALID, "n must be in [0, capacity]");
  if (n > 0 && ids == nullptr) return fail(NS_ERR_INVALID, "ids is NULL");
  int32_t* lens = static_cast<int32_t*>(state);
  int32_t* store = const_cast<int32_t*>(hist_state_ids(state, n_slots));
  const unsigned blocks = (unsigned)((n + 255) / 256 > 0 ? ((n + 255) / 256 < 64 ? (n + 255) / 256 : 64) : 1);
  hipLaunchKernelGGL(ns::hist_assign_kernel, dim3(blocks), dim3(256), 0, stream, lens, store, capacity, slot, ids, n);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("hist_assign launch: ") + hipGetErrorString(e));
  return NS_OK;
}

int ns_seeded_uniforms(const uint64_t* seeds, const int64_t* steps, const int32_t* rows, int32_t n, float* uniforms,
                       hipStream_t stream) {
  if (n < 0) return fail(NS_ERR_INVALID, "n must be >= 0");
  if (n == 0) return NS_OK;
  if (seeds == nullptr || steps == nullptr || uniforms == nullptr)
    return fail(NS_ERR_INVALID, "seeds, steps and uniforms must not be NULL");
  hipLaunchKernelGGL(ns::seeded_uniforms_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, seeds, steps,
                     rows, n, uniforms);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("seeded_uniforms launch: ") + hipGetErrorString(e));
  return NS_OK;
}

int ns_hist_append(void* state, int32_t n_slots, int32_t capacity, const int32_t* slots, const int64_t* token_ids,
                   int32_t n, int32_t* overflow, hipStream_t stream) {
  if (state == nullptr) return fail(NS_ERR_INVALID, "state is NULL");
  int rc = hist_state_check(n_slots, capacity);
  if (rc != NS_OK) return rc;
  if (n < 0) return fail(NS_ERR_INVALID, "n < 0");
  if (n == 0) return NS_OK;
  if (slots == nullptr || token_ids == nullptr) return fail(NS_ERR_INVALID, "slots or token_ids is NULL");
  int32_t* lens = static_cast<int32_t*>(state);
  int32_t* store = const_cast<int32_t*>(hist_state_ids(state, n_slots));
  hipLaunchKernelGGL(ns::hist_append_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, lens, store,
                     n_slots, capacity, slots, token_ids, n, overflow);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("hist_append launch: ") + hipGetErrorString(e));
  return NS_OK;
}

static int lm_check(const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight, const void* logits,
                    int64_t ld_logits, int32_t m, int32_t n, int32_t k, bool packed) {
  if (hidden == nullptr || weight == nullptr || logits == nullptr)
    return fail(NS_ERR_INVALID, "hidden, weight or logits is NULL");
  if (m < 0 || n < 0) return fail(NS_ERR_INVALID, "m or n < 0");
  if (k <= 0 || k % ns::LM_KT != 0) return fail(NS_ERR_INVALID, "k must be a positive multiple of 64");
  if (ld_hidden < k || ld_hidden % 8 != 0 || (!packed && (ld_weight < k || ld_weight % 8 != 0)))
    return fail(NS_ERR_INVALID, "ld_hidden and ld_weight must be multiples of 8 and >= k");
  if (ld_logits < n) return fail(NS_ERR_INVALID, "ld_logits < n");
  if (!packed && ld_weight > (int64_t)(0xffffffffu / (2u * ns::LM_NT)))
    return fail(NS_ERR_INVALID, "ld_weight too large (a workgroup's weight rows span 32-bit offsets)");
  if (((uintptr_t)hidden | (uintptr_t)weight) % 16 != 0)
    return fail(NS_ERR_ALIGN, "hidden and weight must be 16-byte aligned");
  return NS_OK;
}

static int lm_launch(const void* hidden, int64_t ld_hidden, int64_t n_hidden, const int64_t* rows, const void* weight,
                     int64_t ld_weight, void* logits, int64_t ld_logits, int32_t m, int32_t n, int32_t k, bool packed,
                     hipStream_t stream) {
  if (n_hidden <= 0) return fail(NS_ERR_INVALID, "n_hidden must be positive");
  if (rows == nullptr && n_hidden < m) return fail(NS_ERR_INVALID, "n_hidden < m without rows");
  // waves along the batch: the fewest that hold it (64 rows each), so small batches keep every
  // wave on products; batches beyond 256 rows take several workgroup rows
  int wm = m <= 64 ? 1 : m <= 128 ? 2 : 4;
  // WM = 4 keeps two weight stages in flight and needs at least two (k >= 128); a smaller k
  // takes workgroup rows of WM = 2 (the same sums in the same order)
  if (wm == 4 && k < 2 * ns::LM_KT) wm = 2;
  const int64_t gy = ((int64_t)m + 64 * wm - 1) / (64 * wm);
  if (gy > 65535) return fail(NS_ERR_INVALID, "m too large");
  ns::LmParams P{static_cast<const uint16_t*>(hidden), ld_hidden, rows, n_hidden, static_cast<const uint16_t*>(weight),
                 packed ? 0 : ld_weight, static_cast<uint16_t*>(logits), ld_logits, m, n, k};
  // batches beyond 64 rows: the column-owner kernel (weight straight into registers), over
  // 256-row (or, up to 128 rows, 128-row) workgroup rows; its hidden loads take 32-bit offsets
  if (packed && m > 64 && n_hidden * ld_hidden * 2 < (int64_t)0xffffffffu) {
    const int tm = m <= 128 ? 4 : 8;
    const int64_t gyc = ((int64_t)m + 32 * tm - 1) / (32 * tm);
    if (gyc > 65535) return fail(NS_ERR_INVALID, "m too large");
    const dim3 gridc((unsigned)((n + ns::LM_NT - 1) / ns::LM_NT), (unsigned)gyc), blockc(ns::LM_THREADS);
    if (tm == 4) hipLaunchKernelGGL((ns::lm_head_cols_kernel<4>), gridc, blockc, 0, stream, P);
    else hipLaunchKernelGGL((ns::lm_head_cols_kernel<8>), gridc, blockc, 0, stream, P);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("lm_head launch: ") + hipGetErrorString(e));
    return NS_OK;
  }
  const dim3 grid((unsigned)((n + ns::LM_NT - 1) / ns::LM_NT), (unsigned)gy), block(ns::LM_THREADS);
  if (packed) {
    if (wm == 1) hipLaunchKernelGGL((ns::lm_head_kernel<1, 4, true>), grid, block, 0, stream, P);
    else if (wm == 2) hipLaunchKernelGGL((ns::lm_head_kernel<2, 3, true>), grid, block, 0, stream, P);
    else hipLaunchKernelGGL((ns::lm_head_kernel<4, 2, true>), grid, block, 0, stream, P);
  } else {
    if (wm == 1) hipLaunchKernelGGL((ns::lm_head_kernel<1, 4, false>), grid, block, 0, stream, P);
    else if (wm == 2) hipLaunchKernelGGL((ns::lm_head_kernel<2, 3, false>), grid, block, 0, stream, P);
    else hipLaunchKernelGGL((ns::lm_head_kernel<4, 2, false>), grid, block, 0, stream, P);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("lm_head launch: ") + hipGetErrorString(e));
  return NS_OK;
}

int ns_lm_head_bf16(const void* hidden, int64_t ld_hidden, int64_t n_hidden, const int64_t* rows, const void* weight,
                    int64_t ld_weight, void* logits, int64_t ld_logits, int32_t m, int32_t n, int32_t k,
                    hipStream_t stream) {
  const int rc = lm_check(hidden, ld_hidden, weight, ld_weight, logits, ld_logits, m, n, k, false);
  if (rc != NS_OK) return rc;
  if (m == 0 || n == 0) return NS_OK;
  return lm_launch(hidden, ld_hidden, n_hidden, rows, weight, ld_weight, logits, ld_logits, m, n, k, false, stream);
}

int ns_lm_head_packed_bytes(int32_t n, int32_t k, uint64_t* bytes) {
  if (bytes == nullptr) return fail(NS_ERR_INVALID, "bytes is NULL");
  if (n < 0) return fail(NS_ERR_INVALID, "n < 0");
  if (k <= 0 || k % ns::LM_KT != 0) return fail(NS_ERR_INVALID, "k must be a positive multiple of 64");
  *bytes = (uint64_t)((n + ns::LM_NT - 1) / ns::LM_NT) * (uint64_t)(k / ns::LM_KT) * (uint64_t)ns::LM_TILE_BYTES;
  return NS_OK;
}

int ns_lm_head_pack_bf16(const void* weight, int64_t ld_weight, int32_t n, int32_t k, void* packed,
                         hipStream_t stream) {
  if (weight == nullptr || packed == nullptr) return fail(NS_ERR_INVALID, "weight or packed is NULL");
  uint64_t bytes = 0;
  int rc = ns_lm_head_packed_bytes(n, k, &bytes);
  if (rc != NS_OK) return rc;
  if (ld_weight < k || ld_weight % 8 != 0) return fail(NS_ERR_INVALID, "ld_weight must be a multiple of 8 and >= k");
  if (((uintptr_t)weight | (uintptr_t)packed) % 16 != 0)
    return fail(NS_ERR_ALIGN, "weight and packed must be 16-byte aligned");
  if (bytes == 0) return NS_OK;
  const uint64_t pieces = bytes / 16;
  hipLaunchKernelGGL(ns::lm_head_pack_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(weight), ld_weight, n, k, static_cast<uint16_t*>(packed));
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("lm_head pack launch: ") + hipGetErrorString(e));
  return NS_OK;
}

int ns_lm_head_bf16_packed(const void* hidden, int64_t ld_hidden, int64_t n_hidden, const int64_t* rows, const void* packed,
                           uint64_t packed_bytes, void* logits, int64_t ld_logits, int32_t m, int32_t n, int32_t k,
                           hipStream_t stream) {
  int rc = lm_check(hidden, ld_hidden, packed, 0, logits, ld_logits, m, n, k, true);
  if (rc != NS_OK) return rc;
  uint64_t want = 0;
  rc = ns_lm_head_packed_bytes(n, k, &want);
  if (rc != NS_OK) return rc;
  if (packed_bytes != want) return fail(NS_ERR_INVALID, "packed_bytes does not match the packed layout of (n, k)");
  if (m == 0 || n == 0) return NS_OK;
  return lm_launch(hidden, ld_hidden, n_hidden, rows, packed, 0, logits, ld_logits, m, n, k, true, stream);
}

const char* ns_last_error(void) { return g_err.c_str(); }

int ns_sample_noalloc(const ns_sample_args* a, hipStream_t stream) {
  if (a == nullptr) return fail(NS_ERR_INVALID, "args is NULL");
  if (a->workspace != nullptr || a->workspace_bytes != 0)
    return fail(NS_ERR_INVALID, "workspace must be NULL: ns_sample_noalloc uses the library's device scratch");
  if (a->n_sample < 0) return fail(NS_ERR_INVALID, "n_sample < 0");
  if (a->n_sample == 0) return NS_OK;
  if (a->vocab <= 0 || a->vocab > NS_MAX_VOCAB)
    return fail(NS_ERR_INVALID, "vocab must be in [1, " + std::to_string(NS_MAX_VOCAB) + "]");
  if (a->dtype != NS_DTYPE_F32 && a->dtype != NS_DTYPE_BF16) return fail(NS_ERR_INVALID, "dtype must be f32 or bf16");
  if (a->max_hist < 0 || a->max_hist > NS_MAX_HISTORY) return fail(NS_ERR_INVALID, "max_hist out of range");
  const bool hist = a->hist_offsets != nullptr || a->hist_state != nullptr;
  const int64_t need = ws_layout(a->n_sample, a->vocab, a->dtype, hist ? a->max_hist : 0).total;
  if (need > (int64_t)NS_NOALLOC_SCRATCH_BYTES)
    return fail(NS_ERR_INVALID, "this call needs " + std::to_string(need) + " bytes of workspace, above the " +
                                    std::to_string((int64_t)NS_NOALLOC_SCRATCH_BYTES) +
                                    "-byte scratch of ns_sample_noalloc (use ns_sample with a workspace)");
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(NS_ERR_INVALID, "device index beyond the scratch table");
  void* ptr = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[dev];
    if (ptr == nullptr) {
      // first call on this device: the array's address here, and its counters cleared (the
      // sampling kernels leave them at zero after every call)
      e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || ptr == nullptr)
        return fail(NS_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
      hipLaunchKernelGGL(ns::scratch_clear_kernel, dim3(1024), dim3(256), 0, stream, static_cast<uint4*>(ptr),
                         (int64_t)(NS_NOALLOC_SCRATCH_BYTES / 16));
      e = hipGetLastError();
      if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("scratch clear launch: ") + hipGetErrorString(e));
      g_scratch_ptr[dev] = ptr;
    }
  }
  ns_sample_args b = *a;
  b.workspace = ptr;
  b.workspace_bytes = (uint64_t)NS_NOALLOC_SCRATCH_BYTES;
  return ns_sample(&b, stream);
}

int ns_sample_lds_bytes(int64_t vocab, int32_t max_hist, int32_t* lds_bytes) {
  if (lds_bytes == nullptr) return fail(NS_ERR_INVALID, "lds_bytes is NULL");
  if (vocab <= 0 || vocab > NS_MAX_VOCAB) return fail(NS_ERR_INVALID, "vocab out of range");
  if (max_hist < 0 || max_hist > NS_MAX_HISTORY) return fail(NS_ERR_INVALID, "max_hist out of range");
  *lds_bytes = (int32_t)lds_layout(vocab, max_hist).total;
  return NS_OK;
}

int ns_sample_workspace_bytes(int32_t n_sample, int64_t vocab, int32_t dtype, int32_t max_hist, uint64_t* bytes) {
  if (bytes == nullptr) return fail(NS_ERR_INVALID, "bytes is NULL");
  if (n_sample < 0) return fail(NS_ERR_INVALID, "n_sample < 0");
  if (vocab <= 0 || vocab > NS_MAX_VOCAB) return fail(NS_ERR_INVALID, "vocab out of range");
  if (dtype != NS_DTYPE_F32 && dtype != NS_DTYPE_BF16) return fail(NS_ERR_INVALID, "dtype must be f32 or bf16");
  if (max_hist < 0 || max_hist > NS_MAX_HISTORY) return fail(NS_ERR_INVALID, "max_hist out of range");
  *bytes = (uint64_t)ws_layout(n_sample, vocab, dtype, max_hist).total;
  return NS_OK;
}

int ns_sample(const ns_sample_args* a, hipStream_t stream) {
  if (a == nullptr) return fail(NS_ERR_INVALID, "args is NULL");
  if (a->n_sample < 0) return fail(NS_ERR_INVALID, "n_sample < 0");
  if (a->n_sample == 0) return NS_OK;
  ns::KParams p{};
  bool has_hist = false;
  int rc = sample_params(a, p, has_hist);
  if (rc != NS_OK) return rc;
  const int32_t mh = has_hist ? a->max_hist : 0;
  const WsLayout L = ws_layout(a->n_sample, a->vocab, a->dtype, mh);
  const LdsLayout ll = lds_layout(a->vocab, mh);
  const int32_t lds = (int32_t)ll.total;
  p.off_bm = ll.off_bm;
  p.off_xl = ll.off_xl;
  p.xcap = ll.xcap;
  p.off_cand = ll.off_cand;
  p.off_hist = ll.off_hist;
  // rows with more distinct history ids than LDS holds keep them in the workspace
  if (L.xg_cap > 0 && a->workspace == nullptr)
    return fail(NS_ERR_INVALID, "max_hist " + std::to_string(mh) + " above " + std::to_string(NS_LDS_HISTORY) +
                                    " needs a workspace (ns_sample_workspace_bytes with max_hist)");
  if (L.xg_cap > 0) {
    if (a->workspace_bytes < (uint64_t)L.total)
      return fail(NS_ERR_INVALID, "workspace of " + std::to_string(a->workspace_bytes) + " bytes, " +
                                      std::to_string(L.total) + " needed (ns_sample_workspace_bytes)");
    if (((uintptr_t)a->workspace % 256) != 0) return fail(NS_ERR_ALIGN, "workspace must be 256-byte aligned");
    p.xl_glob = reinterpret_cast<float*>(static_cast<unsigned char*>(a->workspace) + L.xlong);
    p.xg_cap = L.xg_cap;
  }
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
  DevInfo di;
  rc = device_info(dev, di);
  if (rc != NS_OK) return rc;
  const int max_lds = di.max_lds;
  if (lds > max_lds)
    return fail(NS_ERR_INVALID, "LDS requirement " + std::to_string(lds) + " exceeds device limit " +
                                    std::to_string(max_lds));

  // Path choice.  Per-row mode: one workgroup per row for every row (greedy and small-k
  // rows that fit in registers stream in one pass); a single launch, best once the batch
  // fills the GPU.  Segmented mode: greedy and small-k rows split over 16-byte-chunk
  // segments (a few workgroups per row); rows with top-k off or larger take the wide path
  // over the same segments; the per-row kernel after them for the rest.
  if (a->mode < NS_MODE_AUTO || a->mode > NS_MODE_PER_ROW) return fail(NS_ERR_INVALID, "unknown mode");
  if (a->mode == NS_MODE_SEGMENTED && a->workspace == nullptr)
    return fail(NS_ERR_INVALID, "segmented mode needs a workspace");
  const int n_cu = di.n_cu;
  bool segmented = a->workspace != nullptr && a->mode != NS_MODE_PER_ROW;
  // AUTO: per-row once the batch fills the GPU and rows fit the streaming path's registers;
  // wider rows keep the segment kernel at every batch size
  const bool fits = a->dtype == NS_DTYPE_BF16 ? ns::row_fits<ns::BF16>(a->vocab) : ns::row_fits<ns::F32>(a->vocab);
  if (a->mode == NS_MODE_AUTO &&
      (((int64_t)a->n_sample * 8 >= (int64_t)n_cu * 7 && fits) || a->n_sample > NS_SEG_MAX_ROWS))
    segmented = false;
  // AUTO: a call declared to hold only small-k rows of up to two streaming phases (512 KiB)
  // takes the one-workgroup-per-row top-k kernel at every batch size: a workgroup streams
  // such a row in less time than several workgroups need to hand their shares over
  const int tk_phases = a->dtype == NS_DTYPE_BF16 ? ns::topk_phases<ns::BF16>(a->vocab)
                                                  : ns::topk_phases<ns::F32>(a->vocab);
  if (a->mode == NS_MODE_AUTO && a->row_kinds == (uint32_t)NS_KIND_SMALL_K && tk_phases <= 2) segmented = false;
  // wide path for the rows neither the streaming nor the segment kernels take
  const bool wide = a->workspace != nullptr && a->mode != NS_MODE_PER_ROW && a->n_sample <= NS_WIDE_MAX_ROWS &&
                    (a->row_kinds == 0u || (a->row_kinds & NS_KIND_OTHER) != 0u);
  if (segmented && a->n_sample > NS_SEG_MAX_ROWS)
    return fail(NS_ERR_INVALID, "segmented mode takes at most " + std::to_string(NS_SEG_MAX_ROWS) + " rows");
  // a call declared to hold only small-k rows, which segmented mode would split: one launch
  // of the split-row kernel, each row over S slices merged by its last workgroup
  int32_t sp_cpt = 1, sp_nch = 0;
  const int sp_S = split_geometry(a->n_sample, a->vocab, a->dtype, n_cu, sp_cpt, sp_nch);
  const bool split = segmented && a->row_kinds == (uint32_t)NS_KIND_SMALL_K && a->n_sample <= ns::SP_MAX_ROWS &&
                     sp_S >= 2 && sp_S <= ns::SP_MAXS;
  if (split) {
    segmented = false;
    if (a->workspace_bytes < (uint64_t)L.total)
      return fail(NS_ERR_INVALID, "workspace of " + std::to_string(a->workspace_bytes) + " bytes, " +
                                      std::to_string(L.total) + " needed (ns_sample_workspace_bytes)");
    if (((uintptr_t)a->workspace % 256) != 0) return fail(NS_ERR_ALIGN, "workspace must be 256-byte aligned");
    unsigned char* ws = static_cast<unsigned char*>(a->workspace);
    ns::SplitParams sp{};
    p.status = nullptr;
    sp.p = p;
    sp.lists = reinterpret_cast<uint64_t*>(ws + L.slist);
    sp.meta = reinterpret_cast<ns::SplitMeta*>(ws + L.smeta);
    sp.counters = reinterpret_cast<int32_t*>(ws + L.counters);
    sp.S = sp_S;
    sp.cpt = sp_cpt;
    sp.nch = sp_nch;
    const dim3 g((unsigned)(((int64_t)a->n_sample + 7) / 8 * 8 * sp_S)), bs(ns::NT);
    if (a->dtype == NS_DTYPE_BF16) hipLaunchKernelGGL((ns::split_kernel<ns::BF16>), g, bs, lds, stream, sp);
    else hipLaunchKernelGGL((ns::split_kernel<ns::F32>), g, bs, lds, stream, sp);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("split kernel launch: ") + hipGetErrorString(e));
    return NS_OK;
  }
  if (segmented || wide) {
    if (a->workspace_bytes < (uint64_t)L.total)
      return fail(NS_ERR_INVALID, "workspace of " + std::to_string(a->workspace_bytes) + " bytes, " +
                                      std::to_string(L.total) + " needed (ns_sample_workspace_bytes)");
    if (((uintptr_t)a->workspace % 256) != 0) return fail(NS_ERR_ALIGN, "workspace must be 256-byte aligned");
  }
  p.fast = 1;
  p.status = nullptr;

  // 1) segment kernel: greedy and small-k rows (launched with the wide path's first pass
  //    when both run)
  ns::SegParams seg_args{};
  if (segmented) {
    const int64_t S = seg_count(a->vocab, a->dtype);
    if (S > ns::MAX_SEGS) return fail(NS_ERR_INVALID, "vocab too large for the segment kernel");
    const int64_t groups = ((int64_t)a->n_sample + 7) / 8;
    const int64_t nblk = groups * 8 * S;
    if (nblk > 0x7fffffffLL) return fail(NS_ERR_INVALID, "too many rows for one launch");
    unsigned char* ws = static_cast<unsigned char*>(a->workspace);
    ns::SegParams s{};
    s.logits = a->logits;
    s.row_stride = a->row_stride;
    s.vocab = a->vocab;
    s.n_rows_total = a->n_rows_total;
    s.sample_idx = a->sample_idx;
    s.temperature = a->temperature;
    s.top_k = a->top_k;
    s.top_p = a->top_p;
    s.penalty = a->rep_penalty;
    s.pen_rcp = p.pen_rcp;
    s.hist_off = a->hist_offsets;
    s.hist_ids = p.hist_ids;
    s.hist_slot = p.hist_slot;
    s.hist_len = p.hist_len;
    s.hist_nslots = a->hist_n_slots;
    s.hist_cap = a->hist_capacity;
    s.uniforms = a->uniforms;
    s.out_ids = p.out_ids;
    s.out_probs = a->out_probs;
    s.out_info = a->out_info;
    s.n_sample = a->n_sample;
    s.S = (int32_t)S;
    s.counters = reinterpret_cast<int32_t*>(ws + L.counters);
    s.status = reinterpret_cast<int32_t*>(ws + L.status);
    s.stats = reinterpret_cast<ns::SegStat*>(ws + L.stats);
    s.cand = reinterpret_cast<uint64_t*>(ws + L.cand);
    p.status = s.status;
    seg_args = s;
    if (!wide) {
      const dim3 g((unsigned)nblk), bs(ns::SNT);
      if (a->dtype == NS_DTYPE_BF16) hipLaunchKernelGGL((ns::segment_kernel<ns::BF16>), g, bs, 0, stream, s);
      else hipLaunchKernelGGL((ns::segment_kernel<ns::F32>), g, bs, 0, stream, s);
      e = hipGetLastError();
      if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("segment kernel launch: ") + hipGetErrorString(e));
    }
  }

  // 2) wide path: rows with top-k off or k > 64, each over the segment workgroups of the
  //    whole GPU; rows it cannot plan keep status 1
  if (wide) {
    const int64_t S = seg_count(a->vocab, a->dtype);
    if (S > ns::MAX_SEGS) return fail(NS_ERR_INVALID, "vocab too large for the segment workgroups");
    const int64_t nblk = ((int64_t)a->n_sample + 7) / 8 * 8 * S;
    unsigned char* ws = static_cast<unsigned char*>(a->workspace);
    ns::WideParams w{};
    w.logits = a->logits;
    w.row_stride = a->row_stride;
    w.vocab = a->vocab;
    w.n_rows_total = a->n_rows_total;
    w.sample_idx = a->sample_idx;
    w.temperature = a->temperature;
    w.top_k = a->top_k;
    w.top_p = a->top_p;
    w.penalty = a->rep_penalty;
    w.pen_rcp = p.pen_rcp;
    w.hist_off = a->hist_offsets;
    w.hist_ids = p.hist_ids;
    w.hist_slot = p.hist_slot;
    w.hist_len = p.hist_len;
    w.hist_nslots = a->hist_n_slots;
    w.hist_cap = a->hist_capacity;
    w.uniforms = a->uniforms;
    w.out_ids = p.out_ids;
    w.out_probs = a->out_probs;
    w.out_info = a->out_info;
    w.n_sample = a->n_sample;
    w.S = (int32_t)S;
    w.init_status = 1;
    w.counters = reinterpret_cast<int32_t*>(ws + L.counters);
    w.status = reinterpret_cast<int32_t*>(ws + L.status);
    w.rows = reinterpret_cast<ns::WideRow*>(ws + L.wrow);
    w.segs = reinterpret_cast<ns::WideSeg*>(ws + L.stats);
    w.shist = reinterpret_cast<uint64_t*>(ws + L.shist);
    w.cand = reinterpret_cast<uint64_t*>(ws + L.cand);
    p.status = w.status;
    const dim3 g((unsigned)nblk), bs(ns::SNT);
    const bool bf = a->dtype == NS_DTYPE_BF16;
    if (segmented) {
      if (bf) hipLaunchKernelGGL((ns::segwide_kernel<ns::BF16>), g, bs, 0, stream, seg_args, w);
      else hipLaunchKernelGGL((ns::segwide_kernel<ns::F32>), g, bs, 0, stream, seg_args, w);
    } else {
      if (bf) hipLaunchKernelGGL((ns::wide_stats_kernel<ns::BF16>), g, bs, 0, stream, w);
      else hipLaunchKernelGGL((ns::wide_stats_kernel<ns::F32>), g, bs, 0, stream, w);
    }
    if (bf) hipLaunchKernelGGL((ns::wide_cut_kernel<ns::BF16>), g, bs, 0, stream, w);
    else hipLaunchKernelGGL((ns::wide_cut_kernel<ns::F32>), g, bs, 0, stream, w);
    // 3) one workgroup per row: the wide rows' final step, and every row the launches above
    //    left, in one launch (the wide step's LDS and the per-row code's share one region)
    const dim3 gr((unsigned)a->n_sample), br(ns::NT);
    const int32_t wlds = (int32_t)sizeof(ns::WideSmemCut) + 16;   // the wide step, and one word past it
    const int32_t flds = lds > wlds ? lds : wlds;
    if (flds > max_lds)
      return fail(NS_ERR_INVALID, "LDS requirement " + std::to_string(flds) + " exceeds device limit " +
                                      std::to_string(max_lds));
    if (bf) hipLaunchKernelGGL((ns::final_kernel<ns::BF16>), gr, br, flds, stream, p, w);
    else hipLaunchKernelGGL((ns::final_kernel<ns::F32>), gr, br, flds, stream, p, w);
    if (a->out_probs != nullptr) {
      // every token's probability of the rows the wide path drew (after their final step)
      if (bf) hipLaunchKernelGGL((ns::wide_probs_kernel<ns::BF16>), g, bs, 0, stream, w);
      else hipLaunchKernelGGL((ns::wide_probs_kernel<ns::F32>), g, bs, 0, stream, w);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("wide kernel launch: ") + hipGetErrorString(e));
    return NS_OK;
  }

  // 3) one workgroup per row: every other row, and rows the segment kernel deferred.  A call
  //    declared to hold only small-k rows, with no kernel before this one, takes the kernel
  //    that requests each row at entry.
  const dim3 grid((unsigned)a->n_sample), block(ns::NT);
  const bool bf = a->dtype == NS_DTYPE_BF16;
  const bool topk = !segmented && !wide && a->row_kinds == (uint32_t)NS_KIND_SMALL_K && tk_phases <= 2;
  if (topk && tk_phases <= 1) {
    if (bf) hipLaunchKernelGGL((ns::topk_kernel<ns::BF16, 1>), grid, block, lds, stream, p);
    else hipLaunchKernelGGL((ns::topk_kernel<ns::F32, 1>), grid, block, lds, stream, p);
  } else if (topk) {
    if (bf) hipLaunchKernelGGL((ns::topk_kernel<ns::BF16, 2>), grid, block, lds, stream, p);
    else hipLaunchKernelGGL((ns::topk_kernel<ns::F32, 2>), grid, block, lds, stream, p);
  } else if (bf) {
    hipLaunchKernelGGL((ns::sample_kernel<ns::BF16>), grid, block, lds, stream, p);
  } else {
    hipLaunchKernelGGL((ns::sample_kernel<ns::F32>), grid, block, lds, stream, p);
  }
  e = hipGetLastError();
  if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("kernel launch: ") + hipGetErrorString(e));
  return NS_OK;
}

int ns_debug_scaled(const ns_sample_args* a, int32_t formula, float* out, int64_t ld_out, hipStream_t stream) {
  if (a == nullptr) return fail(NS_ERR_INVALID, "args is NULL");
  if (a->n_sample < 0) return fail(NS_ERR_INVALID, "n_sample < 0");
  if (a->n_sample == 0) return NS_OK;
  if (formula < ns::DBG_STREAM || formula > ns::DBG_GENERAL) return fail(NS_ERR_INVALID, "unknown formula");
  if (out == nullptr) return fail(NS_ERR_INVALID, "out is NULL");
  if (ld_out < a->vocab) return fail(NS_ERR_INVALID, "ld_out < vocab");
  ns::KParams p{};
  bool has_hist = false;
  const int rc = sample_params(a, p, has_hist);
  if (rc != NS_OK) return rc;
  const size_t lds = (size_t)((a->vocab + 31) / 32) * 4;
  const dim3 grid((unsigned)a->n_sample), block(1024);
  if (a->dtype == NS_DTYPE_BF16)
    hipLaunchKernelGGL((ns::debug_scaled_kernel<ns::BF16>), grid, block, lds, stream, p, formula, out, ld_out);
  else
    hipLaunchKernelGGL((ns::debug_scaled_kernel<ns::F32>), grid, block, lds, stream, p, formula, out, ld_out);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("debug kernel launch: ") + hipGetErrorString(e));
  return NS_OK;
}

}  // extern "C"
