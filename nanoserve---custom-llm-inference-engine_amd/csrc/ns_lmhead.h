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
// k stage, the stage's tile [LM_NT rows][LM_KT] bf16 as 32 contiguous KB, in the order the
// kernel reads it; rows past n are zero.  Each stage is then one contiguous 32 KB read per
// workgroup instead of 256 pieces of 128 B at the row stride, which HBM serves at a far
// lower rate.
constexpr int LM_TILE_BYTES = LM_NT * LM_KT * 2;

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
  const int q = (int)(rem % (LM_TILE_BYTES / 16));   // 16-byte piece within the tile
  const int r = q >> 3, c = (q & 7) * 8;               // tile row, first k of the piece
  const int64_t v = b * LM_NT + r;
  lm_u32x4 x = {0u, 0u, 0u, 0u};
  if (v < n) x = *reinterpret_cast<const lm_u32x4*>(w + v * ldw + (int64_t)st * LM_KT + c);
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
    woff[j] = PACKED ? (uint32_t)((tr + 64 * j) * (LM_KT * 2) + tp * 16) : (uint32_t)((tr + 64 * j) * P.ldw * 2 + tp * 16);
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

}  // namespace ns
