// gfx950 row streaming path for calls whose sampled rows are all top-k rows with
// 1 <= k <= KFAST (the host's NS_KIND_SMALL_K hint), one 1024-thread workgroup per
// row: sampler.py:31-89 for such a row with one HBM pass over it.
//
// Where it differs from row_fast (ns_rowfast.h), which serves rows of any kind:
//   * without sample indices the row's first chunks are requested at entry, before
//     the per-row parameters return; each lane's two history ids are requested as
//     soon as they do, ahead of the rest of its row chunks, so every wave sets its
//     bits (set semantics, sampler.py:34-38) before most of its row data lands and
//     the bitmap is complete at the first barrier after the stream;
//   * the row is read with the non-temporal cache policy;
//   * the bound (the k-th largest of the 128 maxima of 8-lane groups, a lower
//     bound of the k-th largest raw value, mapped through the temperature) is
//     taken by the last wave to finish its share of the row, before the barrier
//     that waits for it, not by one wave after that barrier;
//   * after the barrier each wave stages its chunks that reach the bound in its
//     own LDS slots and expands them, one element per lane, into the candidate
//     list, with no further barrier.
// The candidate list is then ordered by the whole workgroup and drawn by one wave
// (block_finalize_keys), exactly as on the other paths.  Rows this path cannot
// finish (too many candidates, a penalized list short of k) are left to the
// general per-row code, with the same results.
#pragma once

#include <type_traits>

#include "ns_rowfast.h"

namespace ns {

constexpr int TK_CPT = RCPT;                // 16-byte chunks per thread (16)
constexpr int TK_HB = 2;                    // history ids per thread requested with the row
constexpr int TK_EARLY = 4;                 // chunks per thread requested before the parameters return

constexpr int TK_PH = NT * TK_CPT;          // chunks of one phase (one register load per thread)

template <typename T>
__host__ __device__ __forceinline__ bool topk_fits(int64_t V) {
  return row_fits<T>(V);
}

// Phases of TK_PH chunks a row of V tokens takes (the partial chunk counted).  Rows of up to
// two phases are streamed by one workgroup.
template <typename T>
__host__ __device__ __forceinline__ int topk_phases(int64_t V) {
  const int64_t nch = (V + T::EPC - 1) / T::EPC;
  return (int)((nch + TK_PH - 1) / TK_PH);
}

// The NaN guard's uniform row (sampler.py:77-80): probability 1/V for every token and the
// inverse-CDF pick against u over the float64 prefix (i + 1) * fl32(1/V).  Mrep is the value
// reported in the diagnostics (NaN, +inf or -inf).
__device__ __forceinline__ void uniform_row_out(const RowOut& o, float u, int32_t flags, float Mrep) {
  const int64_t V = o.V;
  const float qv = uniform_q(V);
  if (threadIdx.x == 0) put_id(o.out_ids, o.row, uniform_pick(u, qv, V));
  write_info(o, PATH_UNIFORM, (int32_t)V, -__builtin_inff(), (int32_t)V, 0, flags, Mrep, -1);
  if (o.out_probs != nullptr) {
    float* pr = o.out_probs + (int64_t)o.row * V;
    for (int64_t i = threadIdx.x; i < V; i += NT) pr[i] = qv;
  }
}

// A row chunk with the cache policy of its row: non-temporal for one-phase rows (read once,
// staged from registers), the default policy for two-phase rows (their chunks that reach the
// bound are read again, from the L2).
template <int NPH>
__device__ __forceinline__ uint4 topk_load(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  if constexpr (NPH == 1) return buf_load16_nt(r, voff);
  else return buf_load16(r, voff, 0u);
}

// The row's first chunks, requested at kernel entry when the row is known before the
// parameters return (no sample indices): chunk q * NT + t to thread t for q < TK_EARLY.
template <typename T, int NPH = 1>
__device__ __forceinline__ void topk_issue_early(uint4 (&v)[TK_CPT], const unsigned char* rowp, int64_t V) {
  const int64_t nf = V / T::EPC;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(rowp, (uint32_t)(nf < TK_PH ? nf : TK_PH) * 16u);
#pragma unroll
  for (int q = 0; q < TK_EARLY; ++q) {
    v[q] = topk_load<NPH>(r, (uint32_t)(q * NT + threadIdx.x) * 16u);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The bound's key: the k-th largest of the row's group maxima fs (128 per phase; maxima of
// disjoint element groups, so k of them reach it), truncated to its top bits.  One phase:
// 16 bits for bfloat16 (the bits its values carry), 24 for float32.  Two phases: each first-phase
// group is merged with the second-phase group of the same index (the maximum of their union),
// and the key of the k-th of those 128 is truncated to 16 bits, a slightly weaker bound (within
// 2^-7 of the value) for a select of half the votes over two thirds of the bits: it is the
// last wave's serial step after the stream.  Called by one wave.
template <typename T, int NPH>
__device__ __forceinline__ uint32_t topk_bound_key(const float* fs, int lane, int k) {
  if constexpr (NPH == 1) return wave_kth_key<T::SZ == 2 ? 16 : 24>(fkey(fs[lane]), fkey(fs[64 + lane]), k);
  else
    return wave_kth_key<16>(fkey(__builtin_fmaxf(fs[lane], fs[128 + lane])),
                            fkey(__builtin_fmaxf(fs[64 + lane], fs[192 + lane])), k);
}

// A chunk maximum kept as the top 16 bits of its order key, rounded up (the value it stands
// for is >= the maximum, so a chunk is never missed by a test against a bound).
__device__ __forceinline__ uint32_t key16_up(float m) {
  const uint32_t kk = fkey(m);
  return kk >= 0xffff0000u ? 0xffffu : (kk + 0xffffu) >> 16;
}

// The whole row path: every thread of the workgroup calls it.  `v` holds the first TK_EARLY
// chunks when `early` (requested by the caller at entry).  Returns 0 when the row is
// resolved, 1 when it is left to the general per-row code.  NPH = 2: the row streams in two
// phases of TK_PH chunks through the same registers; the first phase's chunk maxima are
// kept (rounded up, 16 bits each), the bound is taken over both phases' group maxima, and
// the chunks of both phases that reach it are read again from the L2.
template <typename T, int NPH = 1>
__device__ __forceinline__ int topk_stream(const RowArgs P, const int row, const unsigned char* rowp,
                                           uint4 (&v)[TK_CPT], const bool early, const int32_t* hp,
                                           const float temp, const int32_t k, const float topp, const float pen,
                                           const float u, const int32_t H, Misc* misc, uint32_t* bm,
                                           uint64_t* cand) {
  constexpr int EPC = T::EPC;
  NS_STAMP_DECL;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wid = wave_id();
  const int64_t V = P.vocab;
  const int nf = (int)(V / EPC);                   // chunks without a token past V
  const int ntail = (int)(V - (int64_t)nf * EPC);  // tokens past the last full chunk
  const uint4* rowv = reinterpret_cast<const uint4*>(rowp);
  const bool pen_on = pen != 1.0f && H > 0;        // sampler.py:33
  const float tdiv = temp > 0.0f ? __builtin_fmaxf(temp, 1e-6f) : 1.0f;   // sampler.py:42
  const float rdiv = 1.0f / tdiv;
  const bool recip = P.pen_rcp != nullptr;
  const float rpen = recip ? P.pen_rcp[row] : 1.0f / pen;
  auto pen_val = [&](float x) -> float { return pen_rn(x, pen, rpen, recip); };
  // the group maxima (128 per phase): two phases use the staging region, free until the bound
  float* fs = NPH == 1 ? reinterpret_cast<float*>(&misc->red) : reinterpret_cast<float*>(cand + HIT_OFF64);
  int32_t* is = reinterpret_cast<int32_t*>(misc->db);    // per-wave NaN / +inf flags
  const RowOut o{P.out_ids, P.out_probs, P.out_info, row, V};
  int32_t flags = 0;

  // LDS set-up: the list padded with keys that sort last, the counters (list length, row
  // flags, arrival tickets), the cleared bitmap.  The barrier
  // orders them before the history bits and the candidates; it comes before the bulk of the
  // row is requested (a wave that has issued all its loads reaches it only as the stream
  // drains, the CU's outstanding requests being limited).
  if (tid < WAVE_CAP) cand[tid] = ~0ull;
  if (tid == 0) { misc->flags = 0; misc->cand_n = 0; misc->ib[0] = 0; }
  if (pen_on) {
    uint4* bm4 = reinterpret_cast<uint4*>(bm);
    const int nbw4 = (int)(((V + 31) / 32 + 3) / 4);   // the bitmap region is padded to 16 bytes
    for (int i = tid; i < nbw4; i += NT) bm4[i] = make_uint4(0u, 0u, 0u, 0u);
  }
  __syncthreads();
  // the first history ids (positions t and NT + t), then the token past the last full chunk
  // at this lane (wave 0), then the rest of the row: chunk q * NT + t to thread t, zeros past
  // the last full chunk.  A wave's loads complete in issue order, so the ids come ahead of
  // all but the few chunks requested at entry.
  if (!early) topk_issue_early<T, NPH>(v, rowp, V);
  int32_t hid[TK_HB];
  {
    const __amdgpu_buffer_rsrc_t rh = make_rsrc(hp, pen_on ? (uint32_t)H * 4u : 0u);
#pragma unroll
    for (int s = 0; s < TK_HB; ++s)
      hid[s] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rh, (int)((uint32_t)(s * NT + tid) * 4u), 0, 2);
  }
  uint32_t xtraw = 0u;
  if (wid == 0 && ntail > 0) xtraw = gather_raw<T>(make_rsrc(rowp, (uint32_t)(V * T::SZ)), nf * EPC + lane);
  __builtin_amdgcn_sched_barrier(0);
  {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(rowp, (uint32_t)(nf < TK_PH ? nf : TK_PH) * 16u);
#pragma unroll
    for (int q = TK_EARLY; q < TK_CPT; ++q) {
      v[q] = topk_load<NPH>(r, (uint32_t)(q * NT + tid) * 16u);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // the history bitmap (set semantics, sampler.py:34-38) as the ids land, ahead of the row
  if (pen_on) {
    bool bad = false;
    for (int base = 0; base < H; base += TK_HB * NT) {
#pragma unroll
      for (int s = 0; s < TK_HB; ++s) {
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
  // Every chunk's NaN-propagating maximum as the row lands (-inf past the full chunks), then
  // the maxima of the wave's 8-lane groups, published with an arrival ticket; the last wave
  // to arrive takes the bound from the 128 published maxima (the barrier below waits for it
  // anyway).  They are maxima of distinct elements, so the k-th largest of them is a lower
  // bound of the row's k-th largest raw value.  Its key is truncated to the bits a bfloat16
  // value carries (24 for float32) and mapped through the temperature
  // (x >= tc  <=>  x / t >= RN(taux / t)).  Measured: a bound over the first 12 to 15 chunks
  // of each thread, taken while the last chunks still stream, is weaker and makes the whole
  // call slower.
  float cm[TK_CPT];
  float gmax = -__builtin_inff();
  bool special = false;
  uint32_t pk[TK_CPT / 2];   // two phases: the first phase's chunk maxima, 16 bits each
  if constexpr (NPH == 2) {
    // the first phase reduced to its chunk maxima, then the second phase, chunks
    // TK_PH + q * NT + t, through the same registers (refilling each register as soon as its
    // first-phase chunk is reduced measured no faster)
    const __amdgpu_buffer_rsrc_t r2 = make_rsrc(rowp + (int64_t)TK_PH * 16, (uint32_t)(nf > TK_PH ? nf - TK_PH : 0) * 16u);
#pragma unroll
    for (int q = 0; q < TK_CPT; ++q) {
      cm[q] = chunk_max<T>(v[q]);
      if ((q + 1) * NT > nf) past_row(cm[q], q * NT + tid, nf);
      special |= !(cm[q] < __builtin_inff());
      gmax = __builtin_fmaxf(gmax, cm[q]);
      if (q & 1) pk[q >> 1] = key16_up(cm[q - 1]) | (key16_up(cm[q]) << 16);
    }
#pragma unroll
    for (int q = 0; q < TK_CPT; ++q) {
      // the default cache policy: this phase's chunks that reach the bound are read again too
      v[q] = buf_load16(r2, (uint32_t)(q * NT + tid) * 16u, 0u);
      __builtin_amdgcn_sched_barrier(0);
    }
    gmax = __builtin_fmaxf(gmax, lane_xor(gmax, 1));
    gmax = __builtin_fmaxf(gmax, lane_xor(gmax, 2));
    gmax = __builtin_fmaxf(gmax, lane_xor(gmax, 4));
    if ((lane & 7) == 0) fs[wid * 8 + (lane >> 3)] = gmax;
    gmax = -__builtin_inff();
  }
  constexpr int C0 = NPH == 2 ? TK_PH : 0;   // first chunk held in the registers now
#pragma unroll
  for (int q = 0; q < TK_CPT; ++q) {
    cm[q] = chunk_max<T>(v[q]);
    if (C0 + (q + 1) * NT > nf) past_row(cm[q], C0 + q * NT + tid, nf);
    special |= !(cm[q] < __builtin_inff());
    gmax = __builtin_fmaxf(gmax, cm[q]);
  }
  gmax = __builtin_fmaxf(gmax, lane_xor(gmax, 1));
  gmax = __builtin_fmaxf(gmax, lane_xor(gmax, 2));
  gmax = __builtin_fmaxf(gmax, lane_xor(gmax, 4));
  if ((lane & 7) == 0) fs[(NPH - 1) * 128 + wid * 8 + (lane >> 3)] = gmax;
  NS_STAMP(1);   // wave 0: its share of the row streamed and reduced
  {
    int ticket = 0;
    if (lane == 0) ticket = __hip_atomic_fetch_add(&misc->ib[0], 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (__builtin_amdgcn_readfirstlane(ticket) == NWAVE - 1) {
      NS_STAMP_LANE(2, lane == 0);   // the last wave to finish its share
      const uint32_t kp = topk_bound_key<T, NPH>(fs, lane, k);
      const float taux = kp <= fkey(-__builtin_inff()) ? -__builtin_inff() : fkey_inv(kp);
      const float b = wave_lower_preimage(taux, tdiv, rdiv);
      NS_STAMP_LANE(7, lane == 0);   // the last wave: the bound taken
      if (lane == 0) misc->fb[0] = b;
    }
  }
  float xt = -__builtin_inff();
  if (wid == 0 && lane < ntail) {
    xt = raw_float<T>(xtraw);
    special |= !(xt < __builtin_inff());
  }
  const bool ws = ballot(special) != 0ull;
  if (lane == 0) is[wid] = ws ? 1 : 0;
  __syncthreads();   // group maxima, flags, the bitmap, the bound
  NS_STAMP(3);
  int spec = 0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) spec |= is[w];
  flags |= misc->flags;
  if (__builtin_expect(spec != 0, 0)) {
    // NaN / +inf among the logits (the penalty keeps both): the softmax is NaN, uniform
    // 1/V (sampler.py:77-80).  Rare: the row is read again to tell NaN from +inf.
    bool nanf = false;
    for (int c = tid; c < nf; c += NT) {
      const uint4 w = rowv[c];
#pragma unroll
      for (int e = 0; e < EPC; ++e) nanf |= T::elem(w, e) != T::elem(w, e);
    }
    if (wid == 0) nanf |= xt != xt;
    const bool anynan = block_any(nanf, &misc->red);
    uniform_row_out(o, u, flags, anynan ? __builtin_nanf("") : __builtin_inff());
    return 0;
  }
  float tc = misc->fb[0];
  // fewer than k finite group maxima (a row of mostly -inf): the general code takes it
  if (__builtin_expect(!(tc > -__builtin_inff()), 0)) { __syncthreads(); return 1; }
  // Chunks whose maximum reaches tc go to the wave's own LDS slots, then the wave expands
  // them into candidates, one element per lane, straight as sort keys (scaled value
  // descending, token id ascending): elements penalized at history positions
  // (sampler.py:37) and kept when they still reach tc.  A penalty >= 1 never raises a value,
  // so every element of the top-k reaches tc after the penalty too; when k of them do, the
  // list holds the whole top-k and its ties.  Every step after the stream runs in all 16
  // waves, four to a SIMD, so it is kept to few instructions per wave.
  uint4* hdat = reinterpret_cast<uint4*>(cand + HIT_OFF64) + wid * HIT_PER_WAVE;
  int32_t* hidx = reinterpret_cast<int32_t*>(cand + HIT_IDX_OFF64) + wid * HIT_PER_WAVE;
  const bool unit_t = tdiv == 1.0f;
  auto take_key = [&](float x, uint32_t id, bool live) {
    if (live && pen_on && ((bm[id >> 5] >> (id & 31)) & 1u)) x = pen_val(x);
    const bool t = live && x >= tc && x > -__builtin_inff();
    const float y = unit_t ? x : div_rn(t ? x : 1.0f, tdiv, rdiv);
    const uint64_t key = desc_key(y, id);
    const uint64_t m = ballot(t);
    if (m == 0ull) return;
    const int leader = __builtin_ctzll(m);
    int base = 0;
    if (lane == leader) base = atomicAdd(&misc->cand_n, __popcll(m));
    base = read_lane(base, leader);
    const int pos = base + lanes_below(m);
    if (t && pos < WAVE_CAP) cand[pos] = key;   // past it: counted only
  };
  // Staging and expansion.  With `reread`, every chunk that reaches tc is staged by index
  // (top bit set) and read again from memory: the row's registers are no longer live.
  auto collect = [&](auto reread) {
    constexpr bool RR = decltype(reread)::value;
    int nh = 0;             // this wave's hit chunks (wave-uniform)
    if constexpr (NPH == 2) {
      // Two phases: every chunk that reaches tc is staged by index (top bit set) and read again
      // from the L2 by the expansion.  Each lane first forms its hit masks of both phases (the
      // first phase against its kept maxima); then one append per round for the lanes that
      // still hold hits, their lowest first (rarely more than one round), instead of a vote
      // per chunk.
      // a kept maximum reaches tc when its 16-bit key reaches tc's key rounded up to 16 bits
      // (the kept keys' low 16 bits are zero; NaN and +inf rows never get here)
      const uint32_t tk16 = (fkey(tc) + 0xffffu) >> 16;
      uint32_t h1 = 0u, h2 = 0u;
#pragma unroll
      for (int q = 0; q < TK_CPT; ++q) {
        h1 |= (((pk[q >> 1] >> ((q & 1) * 16)) & 0xffffu) >= tk16 ? 1u : 0u) << q;
        h2 |= (cm[q] >= tc ? 1u : 0u) << q;   // -inf past the row, and tc > -inf
      }
      while (true) {
        const bool act = (h1 | h2) != 0u;
        const uint64_t m = ballot(act);
        if (m == 0ull) break;
        uint32_t ci = 0u;
        if (act) {
          if (h1 != 0u) {
            ci = (uint32_t)(__builtin_ctz(h1) * NT + tid);
            h1 &= h1 - 1u;
          } else {
            ci = (uint32_t)(C0 + __builtin_ctz(h2) * NT + tid);
            h2 &= h2 - 1u;
          }
        }
        const int pos = nh + lanes_below(m);
        if (act && pos < HIT_PER_WAVE) hidx[pos] = (int32_t)(0x80000000u | ci);
        nh += __popcll(m);
      }
    } else {
#pragma unroll
      for (int q = 0; q < TK_CPT; ++q) {
        const bool hit = cm[q] >= tc;   // -inf past the row, and tc > -inf
        const uint64_t m = ballot(hit);
        if (m != 0ull) {
          const int pos = nh + lanes_below(m);
          if (hit && pos < HIT_PER_WAVE) {
            if constexpr (RR) {
              hidx[pos] = (int32_t)(0x80000000u | (uint32_t)(C0 + q * NT + tid));
            } else {
              hdat[pos] = v[q];
              hidx[pos] = C0 + q * NT + tid;
            }
          }
          nh += __popcll(m);
        }
      }
    }
    NS_STAMP(8);   // wave 0: its chunks staged
    if (__builtin_expect(nh > HIT_PER_WAVE, 0)) {
      // more hit chunks than slots: the count goes past WAVE_CAP and the general code
      // takes the row
      if (lane == 0) atomicAdd(&misc->cand_n, WAVE_CAP + 1);
    } else {
      for (int j = lane; j < ((nh * EPC + 63) & ~63); j += 64) {
        const bool live = j < nh * EPC;
        const int slot = live ? j / EPC : 0, e = j % EPC;
        int32_t ci = hidx[slot];
        uint4 ch;
        if ((NPH == 2 || RR) && ci < 0) {   // staged by index: read again
          ci &= 0x7fffffff;
          ch = rowv[ci];
        } else {
          ch = hdat[slot];
        }
        const float x = elem_sel<T>(ch, e);
        take_key(x, (uint32_t)(ci * EPC + e), live && x >= tc);
      }
    }
    if (ntail > 0 && wid == 0) take_key(xt, (uint32_t)(nf * EPC + lane), lane < ntail);
    NS_STAMP(9);   // wave 0: its candidates listed
  };
  collect(std::false_type{});
  __syncthreads();   // the list complete
  NS_STAMP(4);
  int n = misc->cand_n;
  if (__builtin_expect(n < k && pen_on, 0)) {
    // The penalty took the list under k keys (history tokens among the largest values): the
    // bound again, from the maxima of penalized values (the bitmap is complete), and the list
    // again, every staged chunk read from memory.  At least k penalized values reach the new
    // bound.  Two phases: the first phase is read again whole (its kept maxima are rounded up,
    // not lower bounds); its chunks are then staged against the kept maxima as before, which
    // the penalty never raises.
    if constexpr (NPH == 2) {
      float g1 = -__builtin_inff();
      for (int q0 = 0; q0 < TK_CPT; q0 += 4) {
        uint4 w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = rowv[(q0 + j) * NT + tid];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t hb = T::bits(bm, (q0 + j) * NT + tid);
#pragma unroll
          for (int e = 0; e < EPC; ++e) {
            const float x = T::elem(w[j], e);
            g1 = __builtin_fmaxf(g1, ((hb >> e) & 1u) ? pen_val(x) : x);
          }
        }
      }
      g1 = __builtin_fmaxf(g1, lane_xor(g1, 1));
      g1 = __builtin_fmaxf(g1, lane_xor(g1, 2));
      g1 = __builtin_fmaxf(g1, lane_xor(g1, 4));
      if ((lane & 7) == 0) fs[wid * 8 + (lane >> 3)] = g1;
    }
    // the chunks in registers: those holding history tokens read again for their penalized
    // maxima, four at a time
    float g2 = -__builtin_inff();
#pragma unroll
    for (int q0 = 0; q0 < TK_CPT; q0 += 4) {
      uint32_t hbq[4];
      uint4 w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = C0 + (q0 + j) * NT + tid;
        hbq[j] = c < nf ? T::bits(bm, c) : 0u;
        w[j] = make_uint4(0u, 0u, 0u, 0u);
        if (hbq[j] != 0u) w[j] = rowv[c];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (hbq[j] != 0u) {
          float mx = -__builtin_inff();
#pragma unroll
          for (int e = 0; e < EPC; ++e) {
            const float x = T::elem(w[j], e);
            mx = __builtin_fmaxf(mx, ((hbq[j] >> e) & 1u) ? pen_val(x) : x);
          }
          cm[q0 + j] = mx;
        }
        g2 = __builtin_fmaxf(g2, cm[q0 + j]);
      }
    }
    g2 = __builtin_fmaxf(g2, lane_xor(g2, 1));
    g2 = __builtin_fmaxf(g2, lane_xor(g2, 2));
    g2 = __builtin_fmaxf(g2, lane_xor(g2, 4));
    if ((lane & 7) == 0) fs[(NPH - 1) * 128 + wid * 8 + (lane >> 3)] = g2;
    if (tid < WAVE_CAP) cand[tid] = ~0ull;
    if (tid == 0) misc->cand_n = 0;
    __syncthreads();
    if (wid == 0) {
      const uint32_t kp = topk_bound_key<T, NPH>(fs, lane, k);
      const float taux = kp <= fkey(-__builtin_inff()) ? -__builtin_inff() : fkey_inv(kp);
      if (lane == 0) misc->fb[0] = lower_preimage(taux, tdiv, rdiv);
    }
    __syncthreads();
    tc = misc->fb[0];
    if (tc > -__builtin_inff()) collect(std::true_type{});
    __syncthreads();
    n = misc->cand_n;
  }
  if (__builtin_expect(n > WAVE_CAP || n < k, 0)) { __syncthreads(); return 1; }
  zero_probs(o);
  block_finalize_keys<NT>(cand, cand + WAVE_CAP, n, k, topp < 1.0f, topp, u, row, P.out_ids, P.out_probs, V,
                          P.out_info, flags, n, PATH_WAVE_SET);
  NS_STAMP(6);   // wave 0: drawn and written
  return 0;
}

}  // namespace ns
