// gfx950 split-row path for small batches of top-k rows (1 <= k <= KFAST, the host's
// NS_KIND_SMALL_K hint): sampler.py:31-89 for each row with the row spread over S
// 1024-thread workgroups, so that a batch of a few rows still streams from most of the
// GPU's CUs, in one launch.
//
// Workgroup (row, s) reads its slice of the row once: the history bits of its token range
// (set semantics, sampler.py:34-38), a lower bound of the slice's k-th largest value from
// the maxima of its 8-lane groups, the slice's elements that reach it (penalized at history
// positions, sampler.py:37, scaled by the temperature, :51) as sort keys, and their ranks.
// When the penalty takes the slice's list under k keys, the slice bounds again from the
// maxima of its penalized values (the history bitmap is complete by then) and collects
// again.  It hands over its top-k keys and their ties, in order (at most SP_LIST), with a
// word of flags, then takes an arrival ticket.  The row's k-th largest value is at least
// the slice's k-th largest, so the union of the slices' lists holds the row's top-k set
// and its ties.
//
// The last workgroup of the row to arrive merges the lists: each key's rank in the row is
// its place in its own list plus, for every other list, the number of keys there that sort
// before it (a binary search: the lists are ordered).  The 128 first keys are the ordered
// candidate list of the row, and the top-k, top-p and the draw run on it exactly as on the
// one-workgroup-per-row paths (block_finalize_keys).  Rows this path cannot finish (a list
// longer than SP_LIST, more candidates than WAVE_CAP in a slice, ties of the k-th value past
// the 128 first keys, invalid parameters) are resolved by that workgroup with the general
// per-row code, NaN / +inf rows take the uniform row: results never depend on the path.
#pragma once

#include "ns_topk.h"

namespace ns {

constexpr int SP_MAXS = 4;       // slices per row (measured: more slices make the merge cost more than they save)
constexpr int SP_LIST = 128;     // keys a slice hands over: its top-k and their ties
constexpr int SP_MAX_ROWS = 64;  // rows a split call takes
constexpr int SP_UNION_OFF = 3 * WAVE_CAP;          // merger: the slices' lists (u64 index into cand)
constexpr int SP_SOFF_OFF = 3 * WAVE_CAP - 64;      // merger: each list's keys at or above G (int32)
static_assert(SP_UNION_OFF + SP_MAXS * SP_LIST <= CAP, "the merged lists fit the candidate region");
static_assert(SP_SOFF_OFF >= WAVE_CAP + WAVE_CAP + WAVE_CAP / 2 + WAVE_CAP / 4, "offsets clear of the finaliser's arrays");

enum : int32_t {
  SPF_GENERAL = 1,   // the row needs the general per-row code
  SPF_NAN = 2,       // a NaN among the slice's logits
  SPF_PINF = 4,      // a +inf among the slice's logits (and no NaN)
};

// What a slice hands over besides its keys (8 bytes, written and read as one word).
struct SplitMeta {
  int32_t m;        // keys in the list
  int32_t flags;    // SPF_* bits in the low half, the row's FLAG_* diagnostics bits above
};

struct SplitParams {
  KParams p;           // first: the general per-row code reads it through the argument pointer
  uint64_t* lists;     // [row][slice][SP_LIST] ordered keys
  SplitMeta* meta;     // [row][slice]
  int32_t* counters;   // [row] arrival counters, zero between calls (the merger clears its own)
  int32_t S;           // slices per row: slice s holds chunks [s * nch / S, (s + 1) * nch / S)
  int32_t cpt;         // 16-byte chunks per thread (1..TK_CPT): NT * cpt >= the longest slice
  int32_t nch;         // 16-byte chunks of a row, the partial one included
};

// The slice's work: LDS (misc, bm, cand) of the workgroup, keys to gl.  Returns SPF_* bits;
// m_out is the list's length.  Every thread calls it.
template <typename T>
__device__ __forceinline__ int32_t split_slice(const unsigned char* rowp, const int64_t V, const int c0, const int c1,
                                               const int cpt,
                                               const int32_t* hp, const int32_t H, const float temp, const int32_t k,
                                               const float pen, const float* rcp, Misc* misc, uint32_t* bm,
                                               uint64_t* cand,
                                               uint64_t* gl, int32_t& m_out, int32_t& rflags) {
  constexpr int EPC = T::EPC;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wid = wave_id();
  const int nf = (int)(V / EPC);                   // chunks without a token past V
  const int ntail = (int)(V - (int64_t)nf * EPC);  // tokens past the last full chunk
  const int cf = c1 < nf ? c1 : nf;                // the slice's full chunks: [c0, cf)
  const bool has_tail = ntail > 0 && nf >= c0 && nf < c1;
  const int64_t e0 = (int64_t)c0 * EPC;
  const int64_t e1 = ((int64_t)c1 * EPC < V) ? (int64_t)c1 * EPC : V;
  const bool pen_on = pen != 1.0f && H > 0;        // sampler.py:33
  const float tdiv = temp > 0.0f ? __builtin_fmaxf(temp, 1e-6f) : 1.0f;   // sampler.py:42
  const float rdiv = 1.0f / tdiv;
  const bool recip = rcp != nullptr;
  const float rpen = recip ? *rcp : 1.0f / pen;
  auto pen_val = [&](float x) -> float { return pen_rn(x, pen, rpen, recip); };
  float* fs = reinterpret_cast<float*>(&misc->red);      // the 128 group maxima
  int32_t* is = reinterpret_cast<int32_t*>(misc->db);    // per-wave NaN / +inf flags

  // LDS set-up: the list padded with keys that sort last, the counters, the slice's bitmap.
  // Its barrier comes before the slice is requested (a wave that has issued all its loads
  // reaches a barrier only as they drain).
  if (tid < WAVE_CAP) cand[tid] = ~0ull;
  if (tid == 0) { misc->flags = 0; misc->cand_n = 0; misc->ib[0] = 0; }
  if (pen_on) {
    uint4* bm4 = reinterpret_cast<uint4*>(bm);
    const int nbw4 = (int)(((e1 - e0 + 31) / 32 + 3) / 4);
    for (int i = tid; i < nbw4; i += NT) bm4[i] = make_uint4(0u, 0u, 0u, 0u);
  }
  __syncthreads();
  // the first history ids, the token past the last full chunk at this lane (wave 0), then the
  // slice's chunks (c0 + q * NT + t to thread t, through a buffer range that ends at the
  // slice's last full chunk: zeros past it, with no memory traffic)
  int32_t hid[TK_HB];
  {
    const __amdgpu_buffer_rsrc_t rh = make_rsrc(hp, pen_on ? (uint32_t)H * 4u : 0u);
#pragma unroll
    for (int s = 0; s < TK_HB; ++s)
      hid[s] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rh, (int)((uint32_t)(s * NT + tid) * 4u), 0, 2);
  }
  uint32_t xtraw = 0u;
  if (wid == 0 && has_tail) xtraw = gather_raw<T>(make_rsrc(rowp, (uint32_t)(V * T::SZ)), nf * EPC + lane);
  __builtin_amdgcn_sched_barrier(0);
  uint4 v[TK_CPT];
  {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(rowp + (int64_t)c0 * 16, (uint32_t)(cf > c0 ? cf - c0 : 0) * 16u);
#pragma unroll
    for (int q = 0; q < TK_CPT; ++q) {
      v[q] = make_uint4(0u, 0u, 0u, 0u);
      if (q < cpt) v[q] = buf_load16_nt(r, (uint32_t)(q * NT + tid) * 16u);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // history bits of the slice's token range (set semantics)
  if (pen_on) {
    bool bad = false;
    for (int base = 0; base < H; base += TK_HB * NT) {
#pragma unroll
      for (int s = 0; s < TK_HB; ++s) {
        const int j = base + s * NT + tid;
        const int32_t id = base == 0 ? hid[s] : (j < H ? hp[j] : 0);
        if (j < H) {
          if (id < 0 || (int64_t)id >= V) {
            bad = true;
          } else if ((int64_t)id >= e0 && (int64_t)id < e1) {
            const int32_t l = id - (int32_t)e0;
            atomicOr(&bm[l >> 5], 1u << (l & 31));
          }
        }
      }
    }
    if (bad) atomicOr(&misc->flags, FLAG_BAD_HIST_ID);
  }
  // chunk maxima (-inf past the row), the 8-lane group maxima, and the bound taken by the
  // last wave to arrive: the k-th largest of the 128 group maxima (maxima of distinct
  // elements), truncated to the bits the element type carries, mapped through the
  // temperature (x >= tc  <=>  x / t >= tauy = RN(taux / t))
  float cm[TK_CPT];
  float gmax = -__builtin_inff();
  bool special = false;
#pragma unroll
  for (int q = 0; q < TK_CPT; ++q) {
    cm[q] = -__builtin_inff();
    if (q < cpt) {
      cm[q] = chunk_max<T>(v[q]);
      if (c0 + q * NT + tid >= cf) cm[q] = -__builtin_inff();
    }
    special |= !(cm[q] < __builtin_inff());
    gmax = __builtin_fmaxf(gmax, cm[q]);
  }
  gmax = __builtin_fmaxf(gmax, lane_xor(gmax, 1));
  gmax = __builtin_fmaxf(gmax, lane_xor(gmax, 2));
  gmax = __builtin_fmaxf(gmax, lane_xor(gmax, 4));
  if ((lane & 7) == 0) fs[wid * 8 + (lane >> 3)] = gmax;
  {
    int ticket = 0;
    if (lane == 0) ticket = __hip_atomic_fetch_add(&misc->ib[0], 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (__builtin_amdgcn_readfirstlane(ticket) == NWAVE - 1) {
      const uint32_t kp = wave_kth_key<T::SZ == 2 ? 16 : 24>(fkey(fs[lane]), fkey(fs[64 + lane]), k);
      const float taux = kp <= fkey(-__builtin_inff()) ? -__builtin_inff() : fkey_inv(kp);
      if (lane == 0) misc->fb[0] = lower_preimage(taux, tdiv, rdiv);
    }
  }
  float xt = -__builtin_inff();
  if (wid == 0 && has_tail && lane < ntail) {
    xt = raw_float<T>(xtraw);
    special |= !(xt < __builtin_inff());
  }
  const bool ws = ballot(special) != 0ull;
  if (lane == 0) is[wid] = ws ? 1 : 0;
  __syncthreads();   // group maxima, flags, the bitmap, the bound
  int spec = 0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) spec |= is[w];
  rflags = misc->flags;
  if (spec != 0) {
    // NaN / +inf in the slice (the penalty keeps both): the row is uniform; tell NaN from
    // +inf from the registers
    bool nanf = false;
#pragma unroll
    for (int q = 0; q < TK_CPT; ++q) {
      if (q < cpt && c0 + q * NT + tid < cf) {
#pragma unroll
        for (int e = 0; e < EPC; ++e) nanf |= T::elem(v[q], e) != T::elem(v[q], e);
      }
    }
    nanf |= xt != xt;
    const bool anynan = block_any(nanf, &misc->red);
    return anynan ? SPF_NAN : SPF_PINF;
  }
  float tc = misc->fb[0];
  // chunks reaching tc to the wave's LDS slots, expanded one element per lane into keys
  // (penalized at history positions, kept when they still reach tc), as in topk_stream
  uint4* hdat = reinterpret_cast<uint4*>(cand + HIT_OFF64) + wid * HIT_PER_WAVE;
  int32_t* hidx = reinterpret_cast<int32_t*>(cand + HIT_IDX_OFF64) + wid * HIT_PER_WAVE;
  const bool unit_t = tdiv == 1.0f;
  auto take_key = [&](float x, uint32_t id, bool live) {
    if (live && pen_on) {
      const uint32_t l = id - (uint32_t)e0;
      if ((bm[l >> 5] >> (l & 31)) & 1u) x = pen_val(x);
    }
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
  auto collect = [&]() {
    int nh = 0;
#pragma unroll
    for (int q = 0; q < TK_CPT; ++q) {
      const bool hit = cm[q] >= tc && cm[q] > -__builtin_inff();
      const uint64_t m = ballot(hit);
      if (m != 0ull) {
        const int pos = nh + lanes_below(m);
        if (hit && pos < HIT_PER_WAVE) { hdat[pos] = v[q]; hidx[pos] = c0 + q * NT + tid; }
        nh += __popcll(m);
      }
    }
    if (nh > HIT_PER_WAVE) {
      if (lane == 0) atomicAdd(&misc->cand_n, WAVE_CAP + 1);
    } else {
      for (int j = lane; j < ((nh * EPC + 63) & ~63); j += 64) {
        const bool live = j < nh * EPC;
        const int slot = live ? j / EPC : 0, e = j % EPC;
        const int32_t ci = hidx[slot];
        const uint4 ch = hdat[slot];
        const float x = elem_sel<T>(ch, e);
        take_key(x, (uint32_t)(ci * EPC + e), live && x >= tc);
      }
    }
    if (has_tail && wid == 0) take_key(xt, (uint32_t)(nf * EPC + lane), lane < ntail);
  };
  collect();
  __syncthreads();   // the list complete
  int n = misc->cand_n;
  if (n < k && pen_on && tc > -__builtin_inff()) {
    // The penalty took the list under k keys: the bound again, from maxima of penalized
    // values (the bitmap is complete now), and the list again.  At least k penalized values
    // reach it.
    float gm2 = -__builtin_inff();
#pragma unroll
    for (int q = 0; q < TK_CPT; ++q) {
      const int lc = q * NT + tid;
      if (q < cpt && c0 + lc < cf) {
        const uint32_t hb = T::bits(bm, lc);
        if (hb != 0u) {
          float mx = -__builtin_inff();
#pragma unroll
          for (int e = 0; e < EPC; ++e) {
            const float x = T::elem(v[q], e);
            mx = __builtin_fmaxf(mx, ((hb >> e) & 1u) ? pen_val(x) : x);
          }
          cm[q] = mx;
        }
      }
      gm2 = __builtin_fmaxf(gm2, cm[q]);
    }
    gm2 = __builtin_fmaxf(gm2, lane_xor(gm2, 1));
    gm2 = __builtin_fmaxf(gm2, lane_xor(gm2, 2));
    gm2 = __builtin_fmaxf(gm2, lane_xor(gm2, 4));
    if ((lane & 7) == 0) fs[wid * 8 + (lane >> 3)] = gm2;
    if (tid < WAVE_CAP) cand[tid] = ~0ull;
    if (tid == 0) misc->cand_n = 0;
    __syncthreads();
    if (wid == 0) {
      const uint32_t kp = wave_kth_key<T::SZ == 2 ? 16 : 24>(fkey(fs[lane]), fkey(fs[64 + lane]), k);
      const float taux = kp <= fkey(-__builtin_inff()) ? -__builtin_inff() : fkey_inv(kp);
      if (lane == 0) misc->fb[0] = lower_preimage(taux, tdiv, rdiv);
    }
    __syncthreads();
    tc = misc->fb[0];
    collect();
    __syncthreads();
    n = misc->cand_n;
  }
  // more keys than the list holds; or fewer than k above a finite bound (not reached: the
  // second bound is met by k penalized values)
  if (n > WAVE_CAP || (n < k && tc > -__builtin_inff())) return SPF_GENERAL;
  // the slice's keys in order, then its top-k and their ties to gl
  block_rank_keys<NT>(cand, cand + WAVE_CAP, n);
  __syncthreads();
  const uint64_t* sorted = cand + WAVE_CAP;
  int m = n;
  if (n >= k) {
    const float thr = desc_key_val(sorted[k - 1]);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < WAVE_CAP / 64; ++j) {
      const int i = j * 64 + lane;
      cnt += __popcll(ballot(i < n && desc_key_val(sorted[i < n ? i : 0]) >= thr));
    }
    m = cnt;
  }
  if (m > SP_LIST) return SPF_GENERAL;
  if (wid == 0) {
    if (lane < m) dc_store(gl + lane, sorted[lane]);
    if (64 + lane < m) dc_store(gl + 64 + lane, sorted[64 + lane]);
  }
  m_out = m;
  return 0;
}

template <typename T>
__global__ __launch_bounds__(NT) void split_kernel(const SplitParams SP) {
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int S = SP.S;
  // all slices of a row share blockIdx % 8 (one XCD, one L2 for the row's history)
  const int b = blockIdx.x;
  const int i8 = b >> 3;
  const int rg = i8 / S;
  const int sl = i8 - rg * S;
  const int row = rg * 8 + (b & 7);
  if (row >= SP.p.n_sample) return;
  const int64_t V = SP.p.vocab;
  const float temp = SP.p.temperature[row];
  const int32_t k = SP.p.top_k[row];
  const float topp = SP.p.top_p[row];
  const float pen = SP.p.penalty[row];
  float u = SP.p.uniforms[row];
  const int64_t src = SP.p.sample_idx != nullptr ? SP.p.sample_idx[row] : (int64_t)row;
  int32_t h0 = 0, h1 = 0;
  row_history(SP.p.hist_off, SP.p.hist_slot, SP.p.hist_len, SP.p.hist_nslots, SP.p.hist_cap, row, h0, h1);
  const int32_t H = h1 - h0;
  const bool pen_on = pen != 1.0f && H > 0;
  const bool ok = src >= 0 && src < SP.p.n_rows_total && h0 >= 0 && H >= 0 && H <= MAX_HIST && temp != 0.0f &&
                  k >= 1 && k <= KFAST && (int64_t)k < V && !(pen_on && !(pen > 1.0f && pen <= 3.40282347e38f));
  extern __shared__ __align__(16) unsigned char smem[];
  Misc* misc = reinterpret_cast<Misc*>(smem);
  uint32_t* bm = reinterpret_cast<uint32_t*>(smem + SP.p.off_bm);
  uint64_t* cand = reinterpret_cast<uint64_t*>(smem + SP.p.off_cand);
  uint64_t* gl = SP.lists + ((int64_t)row * S + sl) * SP_LIST;
  int32_t m = 0, rfl = 0, fl = SPF_GENERAL;
  if (ok) {
    const unsigned char* rowp = (const unsigned char*)SP.p.logits + src * SP.p.row_stride * T::SZ;
    const int c0 = (int)((int64_t)sl * SP.nch / S), c1 = (int)((int64_t)(sl + 1) * SP.nch / S);
    fl = split_slice<T>(rowp, V, c0, c1, SP.cpt, SP.p.hist_ids + h0, H, temp, k, pen,
                        SP.p.pen_rcp != nullptr ? SP.p.pen_rcp + row : nullptr, misc, bm,
                        cand, gl, m, rfl);
  }
  // hand over, then the arrival ticket: every wave waits for its device-coherent stores
  // before the barrier, the counter increment follows them
  if (tid == 0)
    dc_store(reinterpret_cast<uint64_t*>(SP.meta + (int64_t)row * S + sl),
             ((uint64_t)(uint32_t)(fl | (rfl << 8)) << 32) | (uint32_t)m);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) misc->ib[1] = arrive_last(&SP.counters[row], S) ? 1 : 0;
  __syncthreads();
  if (misc->ib[1] == 0) return;
  if (tid == 0) __hip_atomic_store(&SP.counters[row], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // ================================ merger ================================
  u = (u >= 0.0f) ? (u < 1.0f ? u : 0x1.fffffep-1f) : 0.0f;
  const RowOut o{SP.p.out_ids, SP.p.out_probs, SP.p.out_info, row, V};
  int32_t* scnt = reinterpret_cast<int32_t*>(cand + SP_SOFF_OFF);   // keys at or above G per list
  uint64_t* uni = cand + SP_UNION_OFF;                                 // list s at uni[s * SP_LIST]
  // one round trip for everything the slices handed over: every slice's word and all of its
  // list slots (slots past a list's length hold keys of earlier calls and are never read)
  const SplitMeta* rm = SP.meta + (int64_t)row * S;
  const uint64_t* rl = SP.lists + (int64_t)row * S * SP_LIST;
  uint64_t w0 = 0ull;
  if (wave_id() == 0 && lane < S) w0 = dc_load(reinterpret_cast<const uint64_t*>(rm + lane));
  for (int f = tid; f < S * SP_LIST; f += NT) uni[f] = dc_load(rl + f);
  if (tid < WAVE_CAP) cand[tid] = ~0ull;
  __syncthreads();
  if (wave_id() == 0) {
    // flags; the prune bound G (the largest k-th key value of a list that holds k keys: no
    // key below it is in the row's top-k set); each list's keys at or above G (a prefix)
    const bool act = lane < S;
    const int32_t ms = act ? (int32_t)(uint32_t)w0 : 0, fls = (int32_t)(uint32_t)(w0 >> 32);
    const int32_t orf = wave_or(fls);
    const uint64_t* ul = uni + lane * SP_LIST;
    const float g = wave_max(act && ms >= k ? desc_key_val(ul[k - 1]) : -__builtin_inff());
    int lo = 0, hi = ms;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (desc_key_val(ul[mid]) >= g) lo = mid + 1; else hi = mid;
    }
    const int nall = wave_sum(lo);
    if (act) scnt[lane] = lo;
    if (lane == 0) {
      misc->ib[2] = orf;
      misc->cand_n = nall;
    }
  }
  __syncthreads();
  const int32_t orf = misc->ib[2] & 0xff;
  const int32_t rflags = misc->ib[2] >> 8;
  if (orf & (SPF_NAN | SPF_PINF)) {
    uniform_row_out(o, u, rflags, (orf & SPF_NAN) ? __builtin_nanf("") : __builtin_inff());
    return;
  }
  if (orf & SPF_GENERAL) {
    row_general<T>((KArgs)__builtin_amdgcn_kernarg_segment_ptr(), row);
    return;
  }
  const int nall = misc->cand_n;   // keys at or above G
  // rank of each key at or above G: its place in its own list plus, in every other list, the
  // keys that sort before it (binary search over that list's prefix); the first WAVE_CAP / 2
  // land in order in cand
  for (int f = tid; f < S * SP_LIST; f += NT) {
    const int s0 = f / SP_LIST, j = f - s0 * SP_LIST;
    if (j >= scnt[s0]) continue;
    const uint64_t key = uni[f];
    int rank = j;
    for (int t = 0; t < S; ++t) {
      if (t == s0) continue;
      const uint64_t* ul = uni + t * SP_LIST;
      int lo = 0, hi = scnt[t];
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (ul[mid] < key) lo = mid + 1; else hi = mid;
      }
      rank += lo;
    }
    if (rank < WAVE_CAP / 2) cand[rank] = key;
  }
  __syncthreads();
  const int n = nall < WAVE_CAP / 2 ? nall : WAVE_CAP / 2;
  bool general = n < k;
  if (!general) {
    // every value at or above the k-th largest must be among the n first
    const float thr = desc_key_val(cand[k - 1]);
    general = nall > n && desc_key_val(cand[n - 1]) >= thr;
  }
  if (general) {
    __syncthreads();
    row_general<T>((KArgs)__builtin_amdgcn_kernarg_segment_ptr(), row);
    return;
  }
  zero_probs(o);
  block_finalize_keys<NT>(cand, cand + WAVE_CAP, n, k, topp < 1.0f, topp, u, row, SP.p.out_ids, SP.p.out_probs, V,
                          SP.p.out_info, rflags, nall, PATH_WAVE_SET);
}

}  // namespace ns
