// gfx950 row streaming path of the one-workgroup-per-row kernel: greedy rows
// and top-k rows with k <= KFAST whose whole row fits in the workgroup's
// registers (RCPT 16-byte chunks per thread: bf16 rows up to 131072 tokens,
// fp32 rows up to 65536).  sampler.py:31-89 for those rows, with one HBM round
// trip per row and no exchange between workgroups:
//   * the history ids are loaded first, then every chunk of the row (chunk
//     q*NT + t to thread t), so the history bitmap (set semantics,
//     sampler.py:34-38) is built while the row is still arriving;
//   * per element only a NaN-propagating chunk maximum is computed, chunk by
//     chunk as the loads land; the unique history positions are gathered and
//     penalized as extra elements, and chunks holding one are no threshold source;
//   * greedy rows: masked maximum and its first index (sampler.py:82-83);
//   * top-k rows: a lower bound of the k-th largest from the 4 largest thread
//     values of every wave (64 values of distinct elements, k-th largest of
//     them), the elements of the chunks reaching it taken from registers into
//     an LDS list, ordered by the whole workgroup (rank counting), then the
//     one-wave top-p / softmax / draw over the top-k prefix.
// Rows whose candidate list outgrows the one-wave capacity (huge tie groups) are
// redone by the general per-row code.
#pragma once

#include "ns_segment.h"

namespace ns {

constexpr int RCPT = 16;               // chunks per thread: the whole row in flight
constexpr int RF_J = 4;                // largest thread values per wave feeding the bound (RF_J * NWAVE >= KFAST)
constexpr int RHB = 2;                 // history ids per thread per batch
static_assert(RF_J * NWAVE == 64, "the bound is selected from one value per lane of wave 0");
static_assert(KFAST <= RF_J * NWAVE, "k-th largest of the per-wave values");

// An opaque copy of a chunk: values derived from it are recomputed rather than
// kept alive from an earlier pass (the row's registers leave no room for them).
__device__ __forceinline__ uint4 fresh(uint4 w) {
  asm volatile("" : "+v"(w.x), "+v"(w.y), "+v"(w.z), "+v"(w.w));
  return w;
}

// bfloat16 bits of an upper bound of x (x itself when x is a bfloat16 value, NaN or inf):
// chunk maxima are kept this way, two per register, to flag chunks that may reach a bound.
__device__ __forceinline__ uint32_t bf16_up(float x) {
  const uint32_t b = __float_as_uint(x);
  uint32_t h = b >> 16;
  if (x > 0.0f && x <= 3.40282347e38f && (b & 0xffffu) != 0u) h += 1u;
  return h;
}
__device__ __forceinline__ float bf16_float(uint32_t h) { return __uint_as_float(h << 16); }

// Wave-aggregated append of (x, id) to the LDS candidate list (32-bit ids); every lane
// of the wave calls it, `take` selects.
__device__ __forceinline__ void cand_push(bool take, float x, uint32_t id, uint64_t* cand, Misc* misc) {
  const uint64_t m = ballot(take);
  if (m == 0ull) return;
  const int leader = __builtin_ctzll(m);
  int base = 0;
  if (lane_id() == leader) base = atomicAdd(&misc->cand_n, __popcll(m));
  base = read_lane(base, leader);
  const int pos = base + lanes_below(m);
  if (take && pos < CAP) cand[pos] = ((uint64_t)__float_as_uint(x) << 32) | id;
}

template <typename T>
__host__ __device__ __forceinline__ bool row_fits(int64_t V) {
  return (V + T::EPC - 1) / T::EPC <= (int64_t)NT * RCPT;
}

// The kernel arguments row_fast reads, passed by value (a reference to the kernel's
// argument block would make the compiler copy it to scratch memory).
struct RowArgs {
  const void* logits;
  int64_t row_stride;
  int64_t vocab;
  const int32_t* hist_ids;
  int64_t* out_ids;
  float* out_probs;
  int32_t* out_info;
};

// Returns 0 when the row is resolved, 1 when its candidate set outgrows the one-wave
// capacity (huge tie groups); the caller then runs the general per-row code.
template <typename T>
__device__ __forceinline__ int row_fast(const RowArgs P, const int row, const int64_t src, const float temp,
                                        const int32_t k, const float topp, const float pen, const float u,
                                        const int32_t h0, const int32_t H, int32_t flags, Misc* misc, uint32_t* bm,
                                        int32_t* xl_id, float* xl_val, uint64_t* cand) {
  constexpr int EPC = T::EPC;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wid = wave_id();
  const int64_t V = P.vocab;
  const int64_t nfull = V / EPC;                  // chunks without a token past V
  const int64_t nchunks = (V + EPC - 1) / EPC;
  const unsigned char* rowp = (const unsigned char*)P.logits + src * P.row_stride * T::SZ;
  const uint4* rowv = reinterpret_cast<const uint4*>(rowp);
  const bool pen_on = pen != 1.0f && H > 0;        // sampler.py:33
  const bool greedy = temp == 0.0f;
  const float tdiv = temp > 0.0f ? __builtin_fmaxf(temp, 1e-6f) : 1.0f;   // sampler.py:42
  const float rdiv = 1.0f / tdiv;
  const float rpen = 1.0f / pen;
  auto pen_val = [&](float x) -> float {
    // sampler.py:37: score * p if score < 0 else score / p (float32, correctly rounded)
    return x < 0.0f ? x * pen : div_rn(x, pen, rpen);
  };
  float* fs = reinterpret_cast<float*>(&misc->red);      // 128 floats of scratch
  int32_t* is = reinterpret_cast<int32_t*>(&misc->red);
  BlockScratch* red = &misc->red;

  // ---- history first, before the row is requested (a load issued while the row
  // streams waits behind it): presence bitmap, unique ids (set semantics), and the
  // gather of the history positions' values
  int U = 0;
  if (pen_on) {
    const int nbw = (int)((V + 31) / 32);
    for (int i = tid; i < nbw; i += NT) bm[i] = 0u;
    if (tid == 0) { misc->xl_n = 0; misc->flags = 0; }
    __syncthreads();
    const int32_t* hp = P.hist_ids + h0;
    bool bad = false;
    for (int base = 0; base < H; base += RHB * NT) {
      int32_t hid[RHB];
#pragma unroll
      for (int s = 0; s < RHB; ++s) {
        const int j = base + s * NT + tid;
        hid[s] = j < H ? hp[j] : 0;
      }
#pragma unroll
      for (int s = 0; s < RHB; ++s) {
        const int32_t id = hid[s];
        bool uniq = false;
        if (base + s * NT + tid < H) {
          if (id < 0 || (int64_t)id >= V) {
            bad = true;
          } else {
            const uint32_t bit = 1u << (id & 31);
            uniq = (atomicOr(&bm[id >> 5], bit) & bit) == 0u;
          }
        }
        const uint64_t m = ballot(uniq);
        if (m != 0ull) {
          int wb = 0;
          if (lane == 0) wb = atomicAdd(&misc->xl_n, __popcll(m));
          wb = read_lane(wb, 0);
          if (uniq) xl_id[wb + lanes_below(m)] = id;
        }
      }
    }
    if (bad) atomicOr(&misc->flags, FLAG_BAD_HIST_ID);
    __syncthreads();
    flags |= misc->flags;
    U = misc->xl_n;
  }
  const float x0 = tid < U ? T::load1(rowp, xl_id[tid]) : 0.0f;   // first NT history values

  // ---- the whole row in flight: buffer loads over the row's full chunks (chunk q*NT + t to
  // thread t); chunks at or past the last full one read zeros and are never used
  const int nf = (int)nfull;
  uint4 v[RCPT];
  {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(rowp, (uint32_t)nf * 16u);
#pragma unroll
    for (int q = 0; q < RCPT; ++q) v[q] = buf_load16(rs, (uint32_t)tid * 16u, (uint32_t)(q * NT * 16));
  }

  // ---- chunk maxima as the loads land (kept: the candidate pass compares them with the
  // bound); threshold sources skip chunks holding history positions
  uint32_t cmp[RCPT / 2];            // chunk maxima (greedy rows: masked), bfloat16 upper bounds
  float tval = -__builtin_inff();
  float gm = -__builtin_inff();      // greedy rows: NaN-propagating masked maximum
  bool nanf = false, pinf = false;
#pragma unroll
  for (int q = 0; q < RCPT; ++q) {
    const int c = q * NT + tid;
    float cmq = chunk_max<T>(v[q]);
    if ((q + 1) * NT > nf && c >= nf) cmq = -__builtin_inff();   // past the last full chunk
    const uint32_t hb = (pen_on && c < nf) ? T::bits(bm, c) : 0u;
    if (hb == 0u) tval = __builtin_fmaxf(tval, cmq);
    else if (greedy) cmq = chunk_max<T>(T::mask(v[q], hb));      // greedy rows: exact masked chunk max
    if (greedy) gm = fmax_nan(gm, cmq);
    if (q & 1) cmp[q >> 1] |= bf16_up(cmq) << 16;
    else cmp[q >> 1] = bf16_up(cmq);
    if (!(cmq <= 3.40282347e38f) && cmq != -__builtin_inff()) {   // NaN or +inf in the chunk (rare)
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        const float x = T::elem(v[q], e);
        if (!((hb >> e) & 1u)) { nanf |= x != x; pinf |= x == __builtin_inff(); }
      }
    }
  }
  // penalized history values: kept in LDS (xl_val), folded into the thread's value
  float xmax = -__builtin_inff();   // NaN-propagating max of this thread's extra values
  for (int i = tid; i < U; i += NT) {
    const float pv = pen_val(i == tid ? x0 : T::load1(rowp, xl_id[i]));
    xl_val[i] = pv;
    xmax = fmax_nan(xmax, pv);
    tval = __builtin_fmaxf(tval, pv);
    nanf |= pv != pv;
    pinf |= pv == __builtin_inff();
  }
  // tokens past the last full chunk (V not a multiple of EPC) join the extras, raw
  if (nfull < nchunks) {
    if (tid == 0) misc->xl_n = U;
    __syncthreads();
    if (wid == 0) {
      const int ntail = (int)(V - nfull * EPC);
      const int64_t id = nfull * EPC + lane;
      const bool act = lane < ntail;
      const bool inhist = act && pen_on && ((bm[id >> 5] >> (id & 31)) & 1u);
      const bool take = act && !inhist;
      const float x = take ? T::load1(rowp, id) : -__builtin_inff();
      const uint64_t m = ballot(take);
      if (take) { xl_id[U + lanes_below(m)] = (int32_t)id; xl_val[U + lanes_below(m)] = x; }
      if (lane == 0) misc->xl_n = U + __popcll(m);
      if (take) {
        xmax = fmax_nan(xmax, x);
        tval = __builtin_fmaxf(tval, x);
        nanf |= x != x;
        pinf |= x == __builtin_inff();
      }
    }
    __syncthreads();
    U = misc->xl_n;
  }
  const RowOut o{P.out_ids, P.out_probs, P.out_info, row, V};

  if (greedy) {
    // masked maximum and its first index (NaN counts as the max, sampler.py:82-83, 88)
    gm = fmax_nan(gm, xmax);
    const float Mx = block_max_nan(gm, red);
    const bool nanm = Mx != Mx;
    int64_t gi = INT64_MAX;
#pragma unroll
    for (int q = 0; q < RCPT; ++q) {
      // chunks of a thread are in ascending token order: the first matching chunk decides
      const int c = q * NT + tid;
      const float cu = bf16_float((cmp[q >> 1] >> (16 * (q & 1))) & 0xffffu);
      if (c < nf && gi == INT64_MAX && (nanm ? (cu != cu) : (cu >= Mx))) {
        const uint32_t hb = pen_on ? T::bits(bm, c) : 0u;
        const uint4 vq = rowv[c];   // re-read (L2)
        const uint4 w = pen_on ? T::mask(vq, hb) : vq;
#pragma unroll
        for (int e = EPC - 1; e >= 0; --e) {
          const float x = T::elem(w, e);
          if ((nanm ? (x != x) : (x == Mx)) && c * EPC + e < V) gi = c * EPC + e;
        }
      }
    }
    for (int i = tid; i < U; i += NT) {
      const float x = xl_val[i];
      if ((nanm ? (x != x) : (x == Mx)) && (int64_t)xl_id[i] < gi) gi = xl_id[i];
    }
    const int64_t best = block_min_i64(gi, red);
    if (tid == 0) P.out_ids[row] = best == INT64_MAX ? 0 : best;
    write_info(o, PATH_GREEDY, 1, -__builtin_inff(), 0, 0, flags, Mx, (int32_t)best);
    return 0;
  }

  // ---- NaN / +inf among the penalized logits: the softmax is NaN, uniform 1/V (sampler.py:77-80)
  {
    const int wf = (ballot(nanf) != 0ull ? 1 : 0) | (ballot(pinf) != 0ull ? 2 : 0);
    if (lane == 0) is[wid] = wf;
  }
  __syncthreads();
  int nanfl = 0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) nanfl |= is[w];
  __syncthreads();
  auto uniform_row = [&](float Mrep) {
    const float qv = (float)(1.0 / (double)V);
    if (tid == 0) {
      const double qd = qv, ud = u;
      int64_t i = (int64_t)(ud / qd);
      while (i > 0 && (double)i * qd > ud) --i;
      while ((double)(i + 1) * qd <= ud && i < V) ++i;
      if (i >= V) i = V - 1;
      P.out_ids[row] = i;
    }
    write_info(o, PATH_UNIFORM, (int32_t)V, -__builtin_inff(), (int32_t)V, 0, flags, Mrep, -1);
    if (P.out_probs != nullptr) {
      float* pr = P.out_probs + (int64_t)row * V;
      for (int64_t i = tid; i < V; i += NT) pr[i] = qv;
    }
  };
  if (nanfl != 0) { uniform_row((nanfl & 1) ? __builtin_nanf("") : __builtin_inff()); return 0; }

  // ---- lower bound of the k-th largest: the k-th largest of the RF_J largest thread values of each wave
  {
    const uint32_t key = wave_sort_u32(~fkey(tval));   // descending
    if (lane < RF_J) fs[wid * RF_J + lane] = fkey_inv(~key);
    __syncthreads();
    if (wid == 0) {
      const uint32_t k2 = wave_sort_u32(~fkey(fs[lane]));
      const float taux = fkey_inv(~read_lane(k2, k - 1));
      if (lane == 0) { fs[64] = taux; misc->cand_n = 0; }
    }
    __syncthreads();
  }
  const float taux = fs[64];
  const float tc = lower_preimage(taux, tdiv, rdiv);   // x >= tc  <=>  x / t >= RN(taux / t)

  // ---- candidates x >= tc: chunks whose maximum reaches tc are re-read (L2) two at a time
  // (the row's registers are free after the chunk pass), then the history positions
  uint32_t fm = 0u;
#pragma unroll
  for (int q = 0; q < RCPT; ++q) {
    const int c = q * NT + tid;
    fm |= (c < nf && bf16_float((cmp[q >> 1] >> (16 * (q & 1))) & 0xffffu) >= tc) ? (1u << q) : 0u;
  }
  {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(rowp, (uint32_t)nf * 16u);
    while (ballot(fm != 0u) != 0ull) {
      const int qa = fm != 0u ? __builtin_ctz(fm) : -1;
      fm &= fm - 1u;
      const int qb = fm != 0u ? __builtin_ctz(fm) : -1;
      fm &= fm - 1u;
      const int ca = qa * NT + tid, cb = qb * NT + tid;
      const uint4 wa = buf_load16(rs, (uint32_t)(qa >= 0 ? ca : 0) * 16u, 0u);
      const uint4 wb = buf_load16(rs, (uint32_t)(qb >= 0 ? cb : 0) * 16u, 0u);
      const uint32_t ha = (pen_on && qa >= 0) ? T::bits(bm, ca) : 0u;
      const uint32_t hb2 = (pen_on && qb >= 0) ? T::bits(bm, cb) : 0u;
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        const float x = T::elem(wa, e);
        cand_push(qa >= 0 && !((ha >> e) & 1u) && x >= tc && x > -__builtin_inff(), x, (uint32_t)ca * EPC + e,
                  cand, misc);
      }
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        const float x = T::elem(wb, e);
        cand_push(qb >= 0 && !((hb2 >> e) & 1u) && x >= tc && x > -__builtin_inff(), x, (uint32_t)cb * EPC + e,
                  cand, misc);
      }
    }
  }
  for (int base = 0; base < U; base += NT) {
    const int i = base + tid;
    const float x = i < U ? xl_val[i] : -__builtin_inff();
    const bool t = x >= tc;
    if (ballot(t) != 0ull) cand_push(t && x > -__builtin_inff(), x, t ? (uint32_t)xl_id[i] : 0u, cand, misc);
  }
  __syncthreads();
  const int n = misc->cand_n;
  if (n == 0) { uniform_row(-__builtin_inff()); return 0; }   // every logit -inf
  if (n <= WAVE_CAP) {
    zero_probs(o);
    block_finalize<NT>(cand, n, k, topp < 1.0f, topp, tdiv, rdiv, u, row, P.out_ids, P.out_probs, V, P.out_info,
                       flags, n, PATH_WAVE_SET);
    return 0;
  }
  __syncthreads();   // every thread has read the candidate count before the caller reuses LDS
  return 1;
}

}  // namespace ns
