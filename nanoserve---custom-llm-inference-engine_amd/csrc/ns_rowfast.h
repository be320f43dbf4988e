// gfx950 row streaming path of the one-workgroup-per-row kernel: greedy rows
// and top-k rows with k <= KFAST whose whole row fits in the workgroup's
// registers (RCPT 16-byte chunks per thread: bf16 rows up to 131072 tokens,
// fp32 rows up to 65536).  sampler.py:31-89 for those rows, with one HBM pass
// over the row and no exchange between workgroups.
//   * Greedy rows: the history (bitmap, unique ids) first, then the row; masked
//     maximum and its first index (sampler.py:82-83).
//   * Top-k rows with a penalty >= 1 (or none): every chunk of the row is
//     requested at once (chunk q*NT + t to thread t), the history ids behind it.
//     Such a penalty never raises a value and keeps NaN / +inf, so the row is
//     processed raw: chunk maxima as the row lands, then a lower bound of the
//     k-th largest (the k-th largest of the maxima of every 8-lane group, by a
//     ballot radix select in one wave while the others build the history bitmap
//     from the ids requested ahead of the row).  Each wave
//     stages its chunks that reach the bound in LDS and expands them into a
//     candidate list, penalized at history positions; a count check confirms the
//     list still covers the top-k.  The list is ordered by the whole workgroup
//     (rank counting) and one wave runs top-p, softmax and the draw over the
//     top-k prefix.
// Rows outside these cases (penalty < 1, huge tie groups, too many staged chunks,
// a failed coverage check) are left to the general per-row code.
#pragma once

#include "ns_segment.h"

namespace ns {

constexpr int RCPT = 16;               // chunks per thread: the whole row in flight
constexpr int RHB = 2;                 // history ids per thread per batch
// LDS staging of the chunks that reach the bound, inside the candidate region (u64
// units): the list uses the first WAVE_CAP entries, its ordered copies the next
// 2 * WAVE_CAP (the id-ordered one over the staging slots, which are dead by then)
constexpr int HIT_PER_WAVE = 48;                               // chunk slots per wave
constexpr int HIT_OFF64 = 2 * WAVE_CAP;                        // 16-byte chunks
constexpr int HIT_IDX_OFF64 = HIT_OFF64 + HIT_PER_WAVE * NWAVE * 2;   // chunk indices
static_assert(KFAST <= 64 && NWAVE * 8 == 128, "the bound: k-th largest of 128 group maxima, k <= 64");
static_assert(HIT_IDX_OFF64 + HIT_PER_WAVE * NWAVE / 2 <= CAP && 3 * WAVE_CAP <= CAP, "candidate region layout");

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

// Raw bits of token id's value (one element) through a buffer descriptor over the row;
// ids outside the descriptor read 0.
template <typename T>
__device__ __forceinline__ uint32_t gather_raw(__amdgpu_buffer_rsrc_t r, int32_t id) {
  if constexpr (T::SZ == 2) return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)((uint32_t)id * 2u), 0, 0);
  else return __builtin_amdgcn_raw_buffer_load_b32(r, (int)((uint32_t)id * 4u), 0, 0);
}
template <typename T>
__device__ __forceinline__ float raw_float(uint32_t b) {
  if constexpr (T::SZ == 2) return __uint_as_float(b << 16);
  else return __uint_as_float(b);
}

// One batch of history ids (NB per thread, id j = base + s*NT + thread): presence bits
// in the LDS bitmap, first occurrences appended to the unique list.  Returns whether
// this thread saw an id outside [0, V).
template <int NB>
__device__ __forceinline__ bool hist_batch(const int32_t (&ids)[NB], int base, int H, int64_t V, uint32_t* bm,
                                           int32_t* xl_id, Misc* misc) {
  const int tid = threadIdx.x;
  const int lane = lane_id();
  bool bad = false;
#pragma unroll
  for (int s = 0; s < NB; ++s) {
    const int32_t id = ids[s];
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
  return bad;
}

// Chunks at or past the row's last full one are read as zeros: their maxima become -inf.
// Called behind a wave-uniform test that only the last chunk rows of a row pass; the empty
// asm keeps that test a branch instead of a select evaluated for every chunk.
__device__ __forceinline__ void past_row(float& m, int c, int nf) {
  asm volatile("");
  if (c >= nf) m = -__builtin_inff();
}

// The k-th largest of the wave's 128 keys (a0, a1 in every lane), truncated to its top NB
// bits: the largest such prefix p with at least k keys >= p, one bit per step from the
// top, counted with ballots.  A lower bound of the k-th largest key.
template <int NB>
__device__ __forceinline__ uint32_t wave_kth_key(uint32_t a0, uint32_t a1, int k) {
  uint32_t p = 0u;
#pragma unroll
  for (int b = 31; b >= 32 - NB; --b) {
    const uint32_t c = p | (1u << b);
    const int cnt = __popcll(ballot(a0 >= c)) + __popcll(ballot(a1 >= c));
    p = cnt >= k ? c : p;
  }
  return p;
}

// Element e (lane-varying) of a chunk held in registers, by selects on the bits of e.
template <typename T>
__device__ __forceinline__ float elem_sel(const uint4& c, int e) {
  if constexpr (T::EPC == 8) {
    const uint32_t lo = (e & 4) ? c.z : c.x, hi = (e & 4) ? c.w : c.y;
    const uint32_t w = (e & 2) ? hi : lo;
    return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
  } else {
    const uint32_t lo = (e & 2) ? c.z : c.x, hi = (e & 2) ? c.w : c.y;
    return __uint_as_float((e & 1) ? hi : lo);
  }
}

template <typename T>
__host__ __device__ __forceinline__ bool row_fits(int64_t V) {
  return (V + T::EPC - 1) / T::EPC <= (int64_t)NT * RCPT;
}

// The row's full chunks into registers, chunk q * NT + t to thread t (chunks past the
// last full one, nf, read zeros), issued in chunk order: a wave's loads complete in issue
// order and the passes over the row take the chunks in that order.
template <typename T>
__device__ __forceinline__ void issue_row(uint4 (&v)[RCPT], const unsigned char* rowp, int nf) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int q = 0; q < RCPT; ++q) {
    v[q] = buf_load16_at(rowp, (uint32_t)nf * 16u, (uint32_t)(q * NT * 16), (uint32_t)tid * 16u);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The kernel arguments row_fast reads, passed by value (a reference to the kernel's
// argument block would make the compiler copy it to scratch memory).
struct RowArgs {
  const void* logits;
  int64_t row_stride;
  int64_t vocab;
  const int32_t* hist_ids;
  IdSink out_ids;
  float* out_probs;
  int32_t* out_info;
  const float* pen_rcp;   // [B] RN(1/p) for the reciprocal penalty, or NULL (division)
};

// Returns 0 when the row is resolved, 1 when it is left to the general per-row code:
// top-k rows with a penalty below 1, candidate sets beyond WAVE_CAP (huge tie groups),
// or penalized candidate sets that no longer cover the top-k.
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
  const bool recip = P.pen_rcp != nullptr;
  const float rpen = recip ? P.pen_rcp[row] : 1.0f / pen;
  auto pen_val = [&](float x) -> float { return pen_rn(x, pen, rpen, recip); };
  float* fs = reinterpret_cast<float*>(&misc->red);      // 128 floats of scratch
  BlockScratch* red = &misc->red;

  const int32_t* hp = P.hist_ids + h0;
  const int nbw = (int)((V + 31) / 32);
  const int nf = (int)nfull;
  const RowOut o{P.out_ids, P.out_probs, P.out_info, row, V};
  auto uniform_row = [&](float Mrep) {
    const float qv = uniform_q(V);
    if (tid == 0) put_id(P.out_ids, row, uniform_pick(u, qv, V));
    write_info(o, PATH_UNIFORM, (int32_t)V, -__builtin_inff(), (int32_t)V, 0, flags, Mrep, -1);
    if (P.out_probs != nullptr) {
      float* pr = P.out_probs + (int64_t)row * V;
      for (int64_t i = tid; i < V; i += NT) pr[i] = qv;
    }
  };
  // top-k rows with a penalty below 1 (or not finite) are left to the general code,
  // before anything touches LDS
  if (!greedy && pen_on && !(pen > 1.0f && pen <= 3.40282347e38f)) return 1;
  if (tid == 0) { misc->xl_n = 0; misc->flags = 0; misc->cand_n = 0; }

  if (greedy) {
    // ---- greedy rows: masked maximum and its first index (NaN counts as the max,
    // sampler.py:82-83, 88).  The history comes first (bitmap and unique ids, set
    // semantics, sampler.py:34-38): requests issued behind the row would be served
    // after it.
    int U = 0;
    if (pen_on) {
      for (int i = tid; i < nbw; i += NT) bm[i] = 0u;
      __syncthreads();
      bool bad = false;
      for (int base = 0; base < H; base += RHB * NT) {
        int32_t ids[RHB];
#pragma unroll
        for (int s = 0; s < RHB; ++s) {
          const int j = base + s * NT + tid;
          ids[s] = j < H ? hp[j] : 0;
        }
        bad |= hist_batch<RHB>(ids, base, H, V, bm, xl_id, misc);
      }
      if (bad) atomicOr(&misc->flags, FLAG_BAD_HIST_ID);
    }
    __syncthreads();
    flags |= misc->flags;
    U = misc->xl_n;
    uint4 v[RCPT];
    issue_row<T>(v, rowp, nf);
    // the first NT history positions' values: raw bits, converted after the row
    const __amdgpu_buffer_rsrc_t rrow = make_rsrc(rowp, (uint32_t)(V * T::SZ));
    const uint32_t x0raw = gather_raw<T>(rrow, U > 0 ? xl_id[tid < U ? tid : 0] : 0);
    uint32_t cmp[RCPT / 2];   // bfloat16 upper bounds of the masked chunk maxima
    float gm = -__builtin_inff();
#pragma unroll
    for (int q = 0; q < RCPT; ++q) {
      const int c = q * NT + tid;
      const uint32_t hb = (pen_on && c < nf) ? T::bits(bm, c) : 0u;
      float cmq = chunk_max<T>(hb != 0u ? T::mask(v[q], hb) : v[q]);
      if ((q + 1) * NT > nf && c >= nf) cmq = -__builtin_inff();   // past the last full chunk
      gm = fmax_nan(gm, cmq);
      if (q & 1) cmp[q >> 1] |= bf16_up(cmq) << 16;
      else cmp[q >> 1] = bf16_up(cmq);
    }
    for (int i = tid; i < U; i += NT) {
      const float pv = pen_val(i == tid ? raw_float<T>(x0raw) : T::load1(rowp, xl_id[i]));
      xl_val[i] = pv;
      gm = fmax_nan(gm, pv);
    }
    // tokens past the last full chunk (V not a multiple of EPC) join the extras, raw
    if (nfull < nchunks) {
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
        if (take) gm = fmax_nan(gm, x);
      }
      __syncthreads();
      U = misc->xl_n;
    }
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
    if (tid == 0) put_id(P.out_ids, row, best == INT64_MAX ? 0 : best);
    write_info(o, PATH_GREEDY, 1, -__builtin_inff(), 0, 0, flags, Mx, (int32_t)best);
    // nothing of this path is left in flight where the top-k path starts (the compiler
    // merges their exits and would otherwise wait for the row there)
    __builtin_amdgcn_s_waitcnt(0);
    return 0;
  }

  // ---- top-k rows with a penalty >= 1 (or none).  Such a penalty never raises a value
  // and keeps NaN and +inf, so the row is processed raw and the candidates are penalized
  // at the end.  The history ids and the tail tokens are requested ahead of the row, so
  // they are in registers when the bitmap is built after the stream (a wave's loads
  // complete in issue order; the few ids hold up the first chunk only).
  int32_t hid[RHB];   // unconditional loads (bounds-checked by the descriptor) keep the counts exact
  {
    const __amdgpu_buffer_rsrc_t rh = make_rsrc(hp, pen_on ? (uint32_t)H * 4u : 0u);
#pragma unroll
    for (int s = 0; s < RHB; ++s)
      hid[s] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rh, (int)((uint32_t)(s * NT + tid) * 4u), 0, 0);
  }
  // tokens past the last full chunk (V not a multiple of EPC): lane l of every wave reads
  // token nfull * EPC + l, zero past the row; wave 0 keeps them
  const int ntail = (int)(V - nfull * EPC);
  const uint32_t xtraw = gather_raw<T>(make_rsrc(rowp, (uint32_t)(V * T::SZ)), (int32_t)(nfull * EPC) + lane);
  __builtin_amdgcn_sched_barrier(0);
  uint4 v[RCPT];
  issue_row<T>(v, rowp, nf);
  // LDS set-up while the row streams, with no barrier: a wave finishes issuing its loads
  // only as the row drains, so a barrier here would hold every wave until then.  The list
  // is padded with keys that sort last and the bitmap cleared; the first barrier below
  // orders both before their use.
  int32_t* is = reinterpret_cast<int32_t*>(misc->db);    // 16 per-wave flags
  if (tid < WAVE_CAP) cand[tid] = ~0ull;
  if (pen_on)
    for (int i = tid; i < nbw; i += NT) bm[i] = 0u;

  // every chunk's NaN-propagating maximum as the row lands (-inf past the full chunks;
  // NaN / +inf only flagged here)
  float cm[RCPT];
  float tval = -__builtin_inff();
  bool special = false;   // NaN or +inf in a chunk
#pragma unroll
  for (int q = 0; q < RCPT; ++q) {
    cm[q] = chunk_max<T>(v[q]);
    if ((q + 1) * NT > nf) past_row(cm[q], q * NT + tid, nf);
    tval = __builtin_fmaxf(tval, cm[q]);
    special |= !(cm[q] < __builtin_inff());
  }
  // the maxima of every 8-lane group (128 values of distinct elements) for the bound
  tval = __builtin_fmaxf(tval, lane_xor(tval, 1));
  tval = __builtin_fmaxf(tval, lane_xor(tval, 2));
  tval = __builtin_fmaxf(tval, lane_xor(tval, 4));
  if ((lane & 7) == 0) fs[wid * 8 + (lane >> 3)] = tval;
  float xt = -__builtin_inff();
  if (wid == 0 && lane < ntail) {
    xt = raw_float<T>(xtraw);
    special |= !(xt < __builtin_inff());
  }
  const bool wspecial = ballot(special) != 0ull;
  if (lane == 0) is[wid] = wspecial ? 1 : 0;
  __syncthreads();   // group maxima, flags, cleared bitmap, padded list
  int spec = 0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) spec |= is[w];
  if (spec != 0) {
    // NaN / +inf among the logits (the penalty keeps both): the softmax is NaN, uniform
    // 1/V (sampler.py:77-80).  Rare: the row is read again to tell NaN from +inf.
    bool nanf = false;
    for (int c = tid; c < nf; c += NT) {
      const uint4 w = rowv[c];
#pragma unroll
      for (int e = 0; e < EPC; ++e) nanf |= T::elem(w, e) != T::elem(w, e);
    }
    if (wid == 0) nanf |= xt != xt;
    const bool anynan = block_any(nanf, red);
    uniform_row(anynan ? __builtin_nanf("") : __builtin_inff());
    return 0;
  }
  // lower bound of the k-th largest raw value: the k-th largest of the group maxima, its
  // key truncated to the bits a bfloat16 value carries (24 for float32)
  if (wid == 0) {
    const uint32_t kp = wave_kth_key<T::SZ == 2 ? 16 : 24>(fkey(fs[lane]), fkey(fs[64 + lane]), k);
    const float taux = kp <= fkey(-__builtin_inff()) ? -__builtin_inff() : fkey_inv(kp);
    // x >= tc  <=>  x / t >= RN(taux / t)
    if (lane == 0) misc->fb[0] = lower_preimage(taux, tdiv, rdiv);
  }
  // the history bitmap (set semantics, sampler.py:34-38), built by every wave while wave 0
  // selects the bound (wave 0 adds its share after it; no wave waits for its atomics before
  // the barrier)
  if (pen_on) {
    bool bad = false;
    for (int base = 0; base < H; base += RHB * NT) {
#pragma unroll
      for (int s = 0; s < RHB; ++s) {
        const int j = base + s * NT + tid;
        const int32_t id = base == 0 ? hid[s] : (j < H ? hp[j] : 0);
        if (j < H) {
          if (id < 0 || (int64_t)id >= V) bad = true;
          else atomicOr(&bm[id >> 5], 1u << (id & 31));
        }
      }
    }
    if (bad) atomicOr(&misc->flags, FLAG_BAD_HIST_ID);
  }
  __syncthreads();   // the bound, the bitmap
  const float tc = misc->fb[0];
  flags |= misc->flags;

  // Chunks whose maximum reaches tc go to the wave's own LDS slots, then the wave expands
  // them into candidates, straight as sort keys (scaled value, token id): elements
  // penalized at history positions (sampler.py:37) and kept when they still reach tc.  A
  // penalty >= 1 never raises a value, so every element of the top-k reaches tc after the
  // penalty too; when k of them do, the list holds the whole top-k and its ties.
  uint4* hdat = reinterpret_cast<uint4*>(cand + HIT_OFF64) + wid * HIT_PER_WAVE;
  int32_t* hidx = reinterpret_cast<int32_t*>(cand + HIT_IDX_OFF64) + wid * HIT_PER_WAVE;
  int nh = 0;             // this wave's hit chunks (wave-uniform)
#pragma unroll
  for (int q = 0; q < RCPT; ++q) {
    const bool hit = cm[q] >= tc;
    const uint64_t m = ballot(hit);
    if (m != 0ull) {
      const int pos = nh + lanes_below(m);
      if (hit && pos < HIT_PER_WAVE) { hdat[pos] = v[q]; hidx[pos] = q * NT + tid; }
      nh += __popcll(m);
    }
  }
  auto take_key = [&](float x, uint32_t id, bool live) {
    if (live && pen_on && ((bm[id >> 5] >> (id & 31)) & 1u)) x = pen_val(x);
    const bool t = live && x >= tc && x > -__builtin_inff();
    // the key before the position, so that its arithmetic overlaps the atomic
    const uint64_t key = desc_key(div_rn(t ? x : 1.0f, tdiv, rdiv), id);
    const uint64_t m = ballot(t);
    if (m == 0ull) return;
    const int leader = __builtin_ctzll(m);
    int base = 0;
    if (lane == leader) base = atomicAdd(&misc->cand_n, __popcll(m));
    base = read_lane(base, leader);
    const int pos = base + lanes_below(m);
    if (t && pos < WAVE_CAP) cand[pos] = key;   // past it: counted only
  };
  if (nh > HIT_PER_WAVE) {
    // more hit chunks than slots: the count goes past WAVE_CAP and the general code
    // takes the row
    if (lane == 0) atomicAdd(&misc->cand_n, WAVE_CAP + 1);
  } else {
    for (int j = lane; j < ((nh * EPC + 63) & ~63); j += 64) {
      const bool live = j < nh * EPC;
      const int slot = live ? j / EPC : 0, e = j % EPC;
      const int32_t ci = hidx[slot];
      const uint4 ch = hdat[slot];
      take_key(elem_sel<T>(ch, e), (uint32_t)(ci * EPC + e), live);
    }
  }
  if (ntail > 0 && wid == 0) take_key(xt, (uint32_t)(nfull * EPC + lane), lane < ntail);
  __syncthreads();   // the list complete
  const int n = misc->cand_n;
  if (n == 0 && !(tc > -__builtin_inff())) { uniform_row(-__builtin_inff()); return 0; }   // every logit -inf
  if (n > WAVE_CAP || (tc > -__builtin_inff() && n < k)) { __syncthreads(); return 1; }
  zero_probs(o);
  block_finalize_keys<NT>(cand, cand + WAVE_CAP, n, k, topp < 1.0f, topp, u, row, P.out_ids, P.out_probs, V,
                          P.out_info, flags, n, PATH_WAVE_SET);
  return 0;
}


}  // namespace ns
