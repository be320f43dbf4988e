// gfx950 lm_head GEMM: the logits producer in front of the sampler.
//
// Replaces, for the sampled positions of a step, the gather, the GEMM and the
// upcast of engine.py:233-236 (hidden.index_select(0, sample_indices), then
// compute_logits(...).float()) and llama.py:136-143 (F.linear(hidden_states,
// embed_tokens.weight), or the untied lm_head):
//
//   logits[r][v] = bf16_rne( sum_k hidden[rows[r]][k] * weight[v][k] )   (fp32 accumulation)
//
// The bf16 rows go to the sampler as they are (it widens each value exactly), so
// the (rows, V) float32 copy is neither written nor read.
//
// Tiling (MFMA v_mfma_f32_32x32x16_bf16, wave64)
//   workgroup: 512 threads (8 waves, two per SIMD so that one wave's LDS waits overlap the
//              other's products), one per CU; LM_NT = 256 vocab rows x 64 WM batch rows,
//              WM = 4, 2 or 1 waves along the batch (the host takes the smallest that holds
//              the batch, so that small batches still give every wave products to do)
//   wave w:    batch rows [64 (w % WM), +64) x vocab rows [32 WM (w / WM), +32 WM): 2 x WM
//              tiles of 32 x 32, 32 WM fp32 accumulators per lane
//   k stages of LM_KT = 64.  Both tiles of a stage -- 256 weight rows x 64 (32 KB, read
//   from HBM once: one pass over the weight in all) and the 64 WM hidden rows x 64 (L2-
//   resident: every workgroup reads all of them) -- are read D stages ahead into registers
//   (D = 2, 3, 4 for WM = 4, 2, 1: as many as the accumulators leave registers for), 8
//   threads per row (128 contiguous bytes), then written to an LDS double buffer from which
//   the waves take their MFMA operands.  The stage barrier orders LDS only, so the
//   prefetches stay in flight across it.
//   Inside a stage the k order is permuted the same way for both operands: at k-step s
//   the lanes of half h (lane / 32) take k = 32h + 8s .. 32h + 8s + 7.  A dot product does
//   not depend on the order of its terms; only the fp32 rounding of the running sum does.
// Batches beyond 64 rows over the packed weight take lm_head_cols_kernel (below): the same
// products in the same order, with each wave owning 32 vocab rows and the whole batch, the
// weight streamed straight into registers and only the hidden tile in LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ns_device.h"

namespace ns {

typedef __bf16 lm_bf16x8 __attribute__((ext_vector_type(8)));
typedef float lm_f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t lm_u32x4 __attribute__((ext_vector_type(4)));

constexpr int LM_THREADS = 512;       // 8 waves
constexpr int LM_NT = 256;            // vocab rows (logit columns) per workgroup
constexpr int LM_MT = 256;            // batch rows per workgroup at most (64 per wave along the batch)
constexpr int LM_KT = 64;             // k per stage
constexpr int LM_PITCH = LM_KT + 8;   // bf16 per LDS row: 144 B, so 16 consecutive rows' 16-byte reads hit distinct banks
constexpr int LM_WL = LM_NT * LM_KT * 2 / 16 / LM_THREADS;   // 16-byte weight loads per thread per stage (4)

struct LmParams {
  const uint16_t* hidden;   // (rows of the hidden tensor, ldh) bf16
  int64_t ldh;
  const int64_t* rows;      // [m] hidden row of each logits row, or NULL: row r
  int64_t n_hidden;         // rows of the hidden tensor: a gathered index outside [0, n_hidden)
                            // reads row 0 and its logits row is written as NaN
  const uint16_t* weight;   // (n, ldw) bf16: out_features x in_features; or the packed tiles
  int64_t ldw;              // (0 for the packed layout)
  uint16_t* logits;         // (m, ldl) bf16
  int64_t ldl;
  int32_t m;
  int32_t n;
  int32_t k;                // multiple of LM_KT
};

// float -> bf16, round to nearest even; a NaN stays a (quiet) NaN
__device__ __forceinline__ uint16_t lm_bf16_rne(float x) {
  uint32_t b = __float_as_uint(x);
  if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x40u);
  b += 0x7fffu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

// Workgroup barrier that orders LDS accesses only: outstanding global loads stay in flight
// (a full barrier would also wait for every load issued ahead).
__device__ __forceinline__ void lm_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Packed weight layout (ns_lm_head_pack_bf16): for each block of LM_NT vocab rows and each
// k stage, the stage's tile [LM_NT rows][LM_KT] bf16 as 32 contiguous KB; rows past n are
// zero.  Each stage is then one contiguous 32 KB read per workgroup instead of 256 pieces of
// 128 B at the row stride, which HBM serves at a far lower rate.  Inside the tile the
// 16-byte pieces are in the order one wave's MFMA B operands take them: for each block of
// 32 rows (one wave's columns in lm_head_cols_kernel), for each k-step s, the 64 lanes'
// pieces (lane l: row l % 32, k = 32 (l / 32) + 8 s .. + 7), so each load instruction of a
// wave reads 1 KB contiguous.
constexpr int LM_TILE_BYTES = LM_NT * LM_KT * 2;

// Piece index, inside its packed tile, of tile row `row` (0..LM_NT-1) and the stage's k chunk c
// (k = 8c .. 8c + 7 of the stage; c = 4 h + s for lane half h and k-step s).
__host__ __device__ __forceinline__ int lm_packed_piece(int row, int c) {
  return (((row >> 5) * 4 + (c & 3)) << 6) + (row & 31) + ((c >> 2) << 5);
}

__global__ void lm_head_pack_kernel(const uint16_t* __restrict__ w, int64_t ldw, int32_t n, int32_t k,
                                    uint16_t* __restrict__ packed) {
  // one thread per 16 bytes of the packed matrix
  const int nst = k / LM_KT;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_block = (int64_t)nst * (LM_TILE_BYTES / 16);
  const int64_t nblk = (n + LM_NT - 1) / LM_NT;
  if (i >= nblk * per_block) return;
  const int64_t b = i / per_block;
  const int64_t rem = i - b * per_block;
  const int st = (int)(rem / (LM_TILE_BYTES / 16));
  const int p = (int)(rem % (LM_TILE_BYTES / 16));   // 16-byte piece within the tile
  // the inverse of lm_packed_piece: row block p / 256, k-step (p / 64) % 4, lane p % 64
  const int l = p & 63;
  const int r = ((p >> 8) << 5) + (l & 31);            // tile row
  const int c = ((l >> 5) << 2) + ((p >> 6) & 3);      // k chunk of the stage
  const int64_t v = b * LM_NT + r;
  lm_u32x4 x = {0u, 0u, 0u, 0u};
  if (v < n) x = *reinterpret_cast<const lm_u32x4*>(w + v * ldw + (int64_t)st * LM_KT + c * 8);
  *reinterpret_cast<lm_u32x4*>(packed + i * 8) = x;
}

template <int WM, int D, bool PACKED>
__global__ __launch_bounds__(LM_THREADS, 1) void lm_head_kernel(const LmParams P) {
  constexpr int MT = 64 * WM;                       // batch rows per workgroup
  constexpr int WN = LM_THREADS / 64 / WM;          // waves along the vocab
  constexpr int NW = LM_NT / WN;                    // vocab rows per wave
  constexpr int JT = NW / 32;                       // 32-row vocab tiles per wave
  constexpr int LM_AL = MT * LM_KT * 2 / 16 / LM_THREADS;   // 16-byte hidden loads per thread per stage
  static_assert(JT >= 1 && LM_AL >= 1, "tiling");
  __shared__ __attribute__((aligned(16))) uint16_t sw[2][LM_NT * LM_PITCH];   // weight tiles
  __shared__ __attribute__((aligned(16))) uint16_t sa[2][MT * LM_PITCH];      // hidden tiles
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * LM_NT;
  const int m0 = blockIdx.y * MT;
  const int wm = wave % WM, wn = wave / WM;      // the wave's 64-row block and vocab share
  const int mw = m0 + wm * 64;                   // this wave's first logits row
  const bool active = mw < P.m;                  // waves whose rows all lie past m skip the products
  const int r32 = lane & 31, h = lane >> 5;

  // stage tiles: thread -> tile rows tid / 8 + 64 j (j < 4), 16-byte piece tid % 8 of the
  // stage's 128 bytes (8 threads read one row's 128 contiguous bytes)
  const int tr = tid >> 3, tp = tid & 7;
  // weight: buffer loads over the workgroup's rows (32-bit offsets; rows past n read as 0),
  // or over the workgroup's packed tiles
  const int nrows = P.n - n0 < LM_NT ? P.n - n0 : LM_NT;
  const int nst = P.k / LM_KT;
  const __amdgpu_buffer_rsrc_t wrs =
      PACKED ? make_rsrc(P.weight + (int64_t)blockIdx.x * nst * (LM_TILE_BYTES / 2), (uint32_t)(nst * LM_TILE_BYTES))
             : make_rsrc(P.weight + (int64_t)n0 * P.ldw, (uint32_t)(nrows * P.ldw * 2));
  uint32_t woff[LM_WL];
#pragma unroll
  for (int j = 0; j < LM_WL; ++j)
    woff[j] = PACKED ? (uint32_t)(lm_packed_piece(tr + 64 * j, tp) * 16) : (uint32_t)((tr + 64 * j) * P.ldw * 2 + tp * 16);
  // hidden: the gathered rows (rows past m read the last row; never stored)
  const uint16_t* asrc[LM_AL];
#pragma unroll
  for (int j = 0; j < LM_AL; ++j) {
    int r = m0 + tr + 64 * j;
    r = r < P.m ? r : P.m - 1;
    int64_t hr = P.rows != nullptr ? P.rows[r] : (int64_t)r;
    hr = hr >= 0 && hr < P.n_hidden ? hr : 0;
    asrc[j] = P.hidden + hr * P.ldh + tp * 8;
  }

  lm_f32x16 acc[2][JT];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < JT; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  lm_u32x4 wr[D][LM_WL], ar[D][LM_AL];   // register stage sets: stage st lives in set st % D

  // the hidden loads first: a wait for them never waits for the weight's HBM loads
  auto load = [&](lm_u32x4 (&a)[LM_AL], lm_u32x4 (&w)[LM_WL], int st) {
    const int ko = st * LM_KT;
#pragma unroll
    for (int j = 0; j < LM_AL; ++j) a[j] = *reinterpret_cast<const lm_u32x4*>(asrc[j] + ko);
#pragma unroll
    for (int j = 0; j < LM_WL; ++j) {
      // streamed once: non-temporal
      const ns_v4u x =
          __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)woff[j], PACKED ? st * LM_TILE_BYTES : ko * 2, 2);
      w[j] = lm_u32x4{x[0], x[1], x[2], x[3]};
    }
  };
  auto store = [&](const lm_u32x4 (&a)[LM_AL], const lm_u32x4 (&w)[LM_WL], int buf) {
#pragma unroll
    for (int j = 0; j < LM_AL; ++j) *reinterpret_cast<lm_u32x4*>(&sa[buf][(tr + 64 * j) * LM_PITCH + tp * 8]) = a[j];
#pragma unroll
    for (int j = 0; j < LM_WL; ++j) *reinterpret_cast<lm_u32x4*>(&sw[buf][(tr + 64 * j) * LM_PITCH + tp * 8]) = w[j];
  };
  auto compute = [&](int buf) {
    const uint16_t* wt = sw[buf] + (wn * NW + r32) * LM_PITCH + 32 * h;
    const uint16_t* at = sa[buf] + (wm * 64 + r32) * LM_PITCH + 32 * h;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      lm_bf16x8 a[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const lm_bf16x8*>(at + 32 * i * LM_PITCH + 8 * s);
#pragma unroll
      for (int j = 0; j < JT; ++j) {
        // one weight operand at a time (JT = 4: the accumulators leave no room for more)
        const lm_bf16x8 b = *reinterpret_cast<const lm_bf16x8*>(wt + 32 * j * LM_PITCH + 8 * s);
#pragma unroll
        for (int i = 0; i < 2; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b, acc[i][j], 0, 0, 0);
      }
    }
  };
  // one stage: stage st + D is issued into the set that held stage st (already in LDS),
  // stage st is computed, stage st + 1 goes to LDS.  D - 1 stages of loads stay in flight
  // across the computation.  The loads and stores are unconditional (stages past the end
  // re-read the last tile, never used): with no branch around them the wait before the
  // stores counts exactly the newer loads in flight.
  auto stage = [&](int st, int d) {
    const int sl = st + D < nst ? st + D : nst - 1;
    load(ar[d], wr[d], sl);
    if (active) compute(st & 1);
    store(ar[(d + 1) % D], wr[(d + 1) % D], (st + 1) & 1);
    lm_lds_barrier();
  };

#pragma unroll
  for (int d = 0; d < D; ++d) load(ar[d], wr[d], d < nst ? d : nst - 1);
  store(ar[0], wr[0], 0);
  lm_lds_barrier();
  int st = 0;
  if constexpr (WM == 4) {
    // at least D stages (the host takes WM = 4 only for k >= 64 D): the pipelined loop runs at
    // least once, and no path around it holds the prefetched stages (there the register
    // allocator, with the 128 accumulators live, would spill them)
    __builtin_assume(nst >= D);
    do {
#pragma unroll
      for (int d = 0; d < D; ++d) stage(st + d, d);
      st += D;
    } while (st + D <= nst);
  } else {
    for (; st + D <= nst; st += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) stage(st + d, d);
    }
  }
#pragma unroll
  for (int d = 0; d < D - 1; ++d)
    if (st + d < nst) stage(st + d, d);

  // 32 x 32 accumulator layout: lane l, element e -> column l % 32, row 8 (e / 4) + 4 (l / 32) + e % 4.
  // Rows whose gathered index lies outside the hidden tensor are written as NaN.
  uint32_t bad = 0u;
  if (P.rows != nullptr) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = mw + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
        if (row < P.m) {
          const int64_t hr = P.rows[row];
          if (hr < 0 || hr >= P.n_hidden) bad |= 1u << (i * 16 + e);
        }
      }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < JT; ++j) {
      const int col = n0 + wn * NW + 32 * j + r32;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = mw + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
        if (row < P.m && col < P.n)
          P.logits[(int64_t)row * P.ldl + col] =
              ((bad >> (i * 16 + e)) & 1u) ? (uint16_t)0x7fc0u : lm_bf16_rne(acc[i][j][e]);
      }
    }
}

typedef __attribute__((address_space(3))) void lm_lds_void;

// One direct-to-LDS load: 16 bytes per lane from the buffer at voff + soff, to LDS at dst + 16 lane
// (dst wave-uniform, a __shared__ address).
__device__ __forceinline__ void lm_load_lds16(__amdgpu_buffer_rsrc_t r, unsigned char* dst, uint32_t voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lm_lds_void*)dst, 16, voff, soff, 0, 0);
}

// Large batches (more than 64 rows) over the packed weight: the column-owner form.  Wave w owns vocab rows
// n0 + 32 w .. + 31 and all MT = 32 TM batch rows of the workgroup (TM tiles of 32 x 32,
// 16 TM accumulators per lane), so each weight piece is used by one wave only: it goes from
// HBM straight into that wave's B operand registers and never through LDS.  A register set
// holds one stage (four k-steps); each k-step's registers are refilled with the stage three
// ahead as soon as its products are issued, so about three stages of weight (96 KB per CU)
// stay in flight.  The hidden tile, shared by the eight waves, goes to LDS by direct-to-LDS
// buffer loads two stages ahead, into a ring of three stage arrays: slot t of a stage
// (16 bytes) holds batch row t / 8's k chunk (t % 8) ^ ((row / 2) % 8), an XOR swizzle under
// which the 16 lanes (16 consecutive rows) of each 256-byte LDS read cycle hit all 64 banks
// once.  The ring's three stages are three arrays and the stage loop is unrolled by three, so
// every LDS access names its array: the compiler then sees that a stage's reads do not touch
// the arrays its direct loads are filling and does not wait for those loads before them.
// Per stage st: this wave's hidden loads of stage st are waited for (the counter form below:
// the loads issued since stay in flight), a barrier makes every wave's share visible (and
// every wave is past stage st - 1's reads, so that array can be refilled), stage st + 2's
// hidden is issued, then stage st's products with the weight refills.  The MFMA operands and
// their order are lm_head_kernel's, so the logits are the same bit for bit.
template <int TM>
__global__ __launch_bounds__(LM_THREADS, 1) void lm_head_cols_kernel(const LmParams P) {
  constexpr int MT = 32 * TM;                   // batch rows per workgroup
  constexpr int SB = MT * LM_KT * 2;            // LDS bytes of one hidden stage
  constexpr int HL = SB / 16 / LM_THREADS;      // direct 16-byte loads per thread per stage
  // loads issued after stage st's hidden loads when stage st is waited for (from stage st + 2
  // on; the prologue's first stages have more): w(st+1), h(st+1), w(st+2)
  constexpr int VMC = 8 + HL;
  constexpr int WAIT = (VMC & 15) | (7 << 4) | (15 << 8) | ((VMC >> 4) << 14);   // vmcnt(VMC) only
  static_assert(HL >= 1 && VMC < 64, "tiling");
  __shared__ __attribute__((aligned(16))) unsigned char sh0[SB];
  __shared__ __attribute__((aligned(16))) unsigned char sh1[SB];
  __shared__ __attribute__((aligned(16))) unsigned char sh2[SB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r32 = lane & 31, h = lane >> 5;
  const int n0 = blockIdx.x * LM_NT;
  const int m0 = blockIdx.y * MT;
  const int nst = P.k / LM_KT;

  // weight (packed): this lane's piece of k-step s of a stage, 1 KB contiguous per wave and
  // k-step (k-step s at + 1 KB)
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc(P.weight + (int64_t)blockIdx.x * nst * (LM_TILE_BYTES / 2), (uint32_t)(nst * LM_TILE_BYTES));
  const uint32_t woff = (uint32_t)(lm_packed_piece(32 * wave + r32, 4 * h) * 16);
  // hidden: this thread's slots j * LM_THREADS + tid of a stage (rows past m read the last row,
  // never stored; a gathered index outside the hidden tensor reads row 0, its logits row is NaN)
  const __amdgpu_buffer_rsrc_t hrs = make_rsrc(P.hidden, (uint32_t)(P.n_hidden * P.ldh * 2));
  uint32_t hoff[HL];
#pragma unroll
  for (int j = 0; j < HL; ++j) {
    const int t = j * LM_THREADS + tid;
    const int mr = t >> 3, c = (t & 7) ^ ((mr >> 1) & 7);
    int r = m0 + mr;
    r = r < P.m ? r : P.m - 1;
    int64_t hr = P.rows != nullptr ? P.rows[r] : (int64_t)r;
    hr = hr >= 0 && hr < P.n_hidden ? hr : 0;
    hoff[j] = (uint32_t)(hr * P.ldh * 2 + c * 16);
  }
  // rows whose gathered index lies outside the hidden tensor (their logits rows are written as
  // NaN): bit rr % 64 of badm[rr / 64] for row m0 + rr, the same in every lane
  uint64_t badm[MT / 64 > 0 ? MT / 64 : 1];
#pragma unroll
  for (int q = 0; q < (MT + 63) / 64; ++q) {
    const int r = m0 + 64 * q + lane;
    bool b = false;
    if (P.rows != nullptr && r < P.m && 64 * q + lane < MT) {
      const int64_t hr = P.rows[r];
      b = hr < 0 || hr >= P.n_hidden;
    }
    badm[q] = __ballot(b);
  }

  lm_f32x16 acc[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;
  lm_bf16x8 wr[3][4];

  // Loads of stages past the last are clamped to it (their data is never used): every stage
  // issues the same loads, so the counter wait counts the same loads every time.
  auto slot = [&](int b) -> unsigned char* { return b == 0 ? sh0 : b == 1 ? sh1 : sh2; };
  auto issue_h = [&](int st, int b) {
    const int sl = st < nst ? st : nst - 1;
    unsigned char* dst = slot(b) + wave * 64 * 16;
#pragma unroll
    for (int j = 0; j < HL; ++j) lm_load_lds16(hrs, dst + j * LM_THREADS * 16, hoff[j], sl * LM_KT * 2);
  };
  auto load_w = [&](int st, int s) -> lm_bf16x8 {
    const int sl = st < nst ? st : nst - 1;
    // streamed once: non-temporal
    const ns_v4u x = __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)(woff + 1024u * s), sl * LM_TILE_BYTES, 2);
    return __builtin_bit_cast(lm_bf16x8, x);
  };
  auto stage = [&](int st, int d) {   // d = st % 3
    __builtin_amdgcn_s_waitcnt(WAIT);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    issue_h(st + 2, (d + 2) % 3);
    __builtin_amdgcn_sched_barrier(0);   // the hidden loads go out first, not after the products
    const unsigned char* ab = slot(d) + r32 * (LM_KT * 2);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int q = ((4 * h + s) ^ ((r32 >> 1) & 7)) << 4;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const lm_bf16x8 a = *reinterpret_cast<const lm_bf16x8*>(ab + i * 4096 + q);
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, wr[d][s], acc[i], 0, 0, 0);
      }
      wr[d][s] = load_w(st + 3, s);   // the k-step's registers, refilled three stages ahead
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // issue order: h0 w0 h1 w1 w2, then at stage st: h(st + 2), and w(st + 3) one k-step at a time
  issue_h(0, 0);
#pragma unroll
  for (int s = 0; s < 4; ++s) wr[0][s] = load_w(0, s);
  issue_h(1, 1);
#pragma unroll
  for (int s = 0; s < 4; ++s) wr[1][s] = load_w(1, s);
#pragma unroll
  for (int s = 0; s < 4; ++s) wr[2][s] = load_w(2, s);
  int st = 0;
  for (; st + 3 <= nst; st += 3) {
    stage(st, 0);
    stage(st + 1, 1);
    stage(st + 2, 2);
  }
  if (st < nst) stage(st, 0);
  if (st + 1 < nst) stage(st + 1, 1);
  // nothing may land in LDS after the workgroup ends
  __builtin_amdgcn_s_waitcnt(0);

  // accumulator layout as in lm_head_kernel: lane l, element e -> column l % 32,
  // row 8 (e / 4) + 4 (l / 32) + e % 4 of tile i
  const int col = n0 + 32 * wave + r32;
  if (col < P.n) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int rr = 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);   // row within the workgroup's rows
        const bool nan_row = (badm[i >> 1] >> (rr & 63)) & 1ull;
        if (m0 + rr < P.m)
          P.logits[(int64_t)(m0 + rr) * P.ldl + col] = nan_row ? (uint16_t)0x7fc0u : lm_bf16_rne(acc[i][e]);
      }
  }
}

}  // namespace ns
