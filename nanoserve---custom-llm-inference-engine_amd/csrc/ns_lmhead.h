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
//              other's products), one per CU; LM_NT = 256 vocab rows x LM_MT = 256 batch rows
//   wave w:    batch rows [64 (w % 4), +64) x vocab rows [128 (w / 4), +128): 2 x 4 tiles
//              of 32 x 32, 128 fp32 accumulators per lane
//   k stages of LM_KT = 64.  Both tiles of a stage -- 256 weight rows x 64 (32 KB, read
//   from HBM once: one pass over the weight in all) and the 256 hidden rows x 64 (32 KB,
//   L2-resident: every workgroup reads all of them) -- are read two stages ahead into
//   registers, 8 threads per row (128 contiguous bytes), then written to an LDS double
//   buffer from which the waves take their MFMA operands.  The stage barrier orders LDS
//   only, so the prefetches stay in flight across it.
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
constexpr int LM_MT = 256;            // batch rows per workgroup, 64 per wave
constexpr int LM_KT = 64;             // k per stage
constexpr int LM_PITCH = LM_KT + 8;   // bf16 per LDS row: 144 B, so 16 consecutive rows' 16-byte reads hit distinct banks
constexpr int LM_WL = LM_NT * LM_KT * 2 / 16 / LM_THREADS;   // 16-byte weight loads per thread per stage (4)
constexpr int LM_AL = LM_MT * LM_KT * 2 / 16 / LM_THREADS;   // 16-byte hidden loads per thread per stage (4)

struct LmParams {
  const uint16_t* hidden;   // (rows of the hidden tensor, ldh) bf16
  int64_t ldh;
  const int64_t* rows;      // [m] hidden row of each logits row, or NULL: row r
  const uint16_t* weight;   // (n, ldw) bf16: out_features x in_features
  int64_t ldw;
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

__global__ __launch_bounds__(LM_THREADS, 1) void lm_head_kernel(const LmParams P) {
  __shared__ __attribute__((aligned(16))) uint16_t sw[2][LM_NT * LM_PITCH];   // weight tiles
  __shared__ __attribute__((aligned(16))) uint16_t sa[2][LM_MT * LM_PITCH];   // hidden tiles
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * LM_NT;
  const int m0 = blockIdx.y * LM_MT;
  const int wm = wave & 3, wn = wave >> 2;       // the wave's 64-row block and 128-column half
  const int mw = m0 + wm * 64;                   // this wave's first logits row
  const bool active = mw < P.m;                  // waves whose rows all lie past m skip the products
  const int r32 = lane & 31, h = lane >> 5;

  // stage tiles: thread -> tile rows tid / 8 + 64 j (j < 4), 16-byte piece tid % 8 of the
  // stage's 128 bytes (8 threads read one row's 128 contiguous bytes)
  const int tr = tid >> 3, tp = tid & 7;
  // weight: buffer loads over the workgroup's rows (32-bit offsets; rows past n read as 0)
  const int nrows = P.n - n0 < LM_NT ? P.n - n0 : LM_NT;
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(P.weight + (int64_t)n0 * P.ldw, (uint32_t)(nrows * P.ldw * 2));
  uint32_t woff[LM_WL];
#pragma unroll
  for (int j = 0; j < LM_WL; ++j) woff[j] = (uint32_t)((tr + 64 * j) * P.ldw * 2 + tp * 16);
  // hidden: the gathered rows (rows past m read the last row; never stored)
  const uint16_t* asrc[LM_AL];
#pragma unroll
  for (int j = 0; j < LM_AL; ++j) {
    int r = m0 + tr + 64 * j;
    r = r < P.m ? r : P.m - 1;
    const int64_t hr = P.rows != nullptr ? P.rows[r] : (int64_t)r;
    asrc[j] = P.hidden + hr * P.ldh + tp * 8;
  }

  lm_f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  lm_u32x4 wx[LM_WL], wy[LM_WL], ax[LM_AL], ay[LM_AL];   // stages of even and odd index
  const int nst = P.k / LM_KT;

  // the hidden loads first: a wait for them never waits for the weight's HBM loads
  auto load = [&](lm_u32x4 (&a)[LM_AL], lm_u32x4 (&w)[LM_WL], int st) {
    const int ko = st * LM_KT;
#pragma unroll
    for (int j = 0; j < LM_AL; ++j) a[j] = *reinterpret_cast<const lm_u32x4*>(asrc[j] + ko);
#pragma unroll
    for (int j = 0; j < LM_WL; ++j) {
      // streamed once: non-temporal
      const ns_v4u x = __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)woff[j], ko * 2, 2);
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
    const uint16_t* wt = sw[buf] + (wn * 128 + r32) * LM_PITCH + 32 * h;
    const uint16_t* at = sa[buf] + (wm * 64 + r32) * LM_PITCH + 32 * h;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      lm_bf16x8 a[2], b[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const lm_bf16x8*>(at + 32 * i * LM_PITCH + 8 * s);
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const lm_bf16x8*>(wt + 32 * j * LM_PITCH + 8 * s);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };
  // one stage: stage st + 2 is issued into the registers that held stage st (already in
  // LDS), stage st is computed, stage st + 1 goes to LDS.  The loads and stores are
  // unconditional (the last two stages re-read the last tile, never used): with no branch
  // around them the wait before the stores counts exactly the newer loads in flight.
  auto stage = [&](int st, lm_u32x4 (&anext)[LM_AL], lm_u32x4 (&wnext)[LM_WL], lm_u32x4 (&athis)[LM_AL],
                   lm_u32x4 (&wthis)[LM_WL]) {
    load(athis, wthis, st + 2 < nst ? st + 2 : nst - 1);
    if (active) compute(st & 1);
    store(anext, wnext, (st + 1) & 1);
    lm_lds_barrier();
  };

  load(ax, wx, 0);
  load(ay, wy, nst > 1 ? 1 : 0);
  store(ax, wx, 0);
  lm_lds_barrier();
  int st = 0;
  for (; st + 1 < nst; st += 2) {
    stage(st, ay, wy, ax, wx);
    stage(st + 1, ax, wx, ay, wy);
  }
  if (st < nst) stage(st, ay, wy, ax, wx);

  // 32 x 32 accumulator layout: lane l, element e -> column l % 32, row 8 (e / 4) + 4 (l / 32) + e % 4
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + wn * 128 + 32 * j + r32;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = mw + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
        if (row < P.m && col < P.n) P.logits[(int64_t)row * P.ldl + col] = lm_bf16_rne(acc[i][j][e]);
      }
    }
}

}  // namespace ns
