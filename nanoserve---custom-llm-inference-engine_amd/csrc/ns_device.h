// Device helpers for the gfx950 token sampler: float keys, wave64 and
// workgroup reductions/scans, exact division by a row-uniform divisor.
//
// Workgroups are 1024 threads = 16 wave64s.  Reductions go through DPP/
// shuffles inside a wave and a small LDS slot array across waves; they never
// use same-address LDS atomics (which serialise across all 1024 lanes).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ns {

constexpr int NT = 1024;          // threads per workgroup
constexpr int NWAVE = NT / 64;    // 16 wave64s

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// Phase stamps of the top-k streaming kernel, in the library built with NS_PHASE_STAMPS
// only (the shipped library compiles them away): the shader clock (s_memtime) at phase
// boundaries of each workgroup, stored to ns_stamp_buf[workgroup * NS_STAMPS + slot] by
// one lane.  No work is skipped; each stamp waits for the wave's outstanding scalar and LDS
// operations, which lengthens the path it sits on slightly.  A function that stamps declares
// NS_STAMP_DECL first: the buffer's address is read once there, not at every stamp.
constexpr int NS_STAMPS = 16;
#ifdef NS_PHASE_STAMPS
__device__ uint64_t* ns_stamp_buf;
#define NS_STAMP_DECL uint64_t* const ns_sb_ = ns::ns_stamp_buf
#define NS_STAMP_LANE(slot, cond)                                                           \
  do {                                                                                       \
    if ((cond) && ns_sb_ != nullptr)                                                         \
      ns_sb_[(int64_t)blockIdx.x * ns::NS_STAMPS + (slot)] = __builtin_amdgcn_s_memtime();  \
  } while (0)
#else
#define NS_STAMP_DECL do { } while (0)
#define NS_STAMP_LANE(slot, cond) do { } while (0)
#endif
#define NS_STAMP(slot) NS_STAMP_LANE(slot, threadIdx.x == 0)

// IEEE-754-2019 maximum/minimum: NaN-propagating (v_maximum3_f32 on gfx950).
__device__ __forceinline__ float fmax_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float fmin_nan(float a, float b) { return __builtin_elementwise_minimum(a, b); }

// Order-preserving uint32 key of a float; -0 and +0 map to the same key (the
// reference compares logits with IEEE ==, where -0 == +0).  NaN is never keyed.
__device__ __forceinline__ uint32_t fkey(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float fkey_inv(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// Sort key ordering (value descending, token id ascending) as an ascending u64.
__device__ __forceinline__ uint64_t desc_key(float y, uint32_t id) {
  return ((uint64_t)(~fkey(y)) << 32) | (uint64_t)id;
}
__device__ __forceinline__ float desc_key_val(uint64_t k) { return fkey_inv(~(uint32_t)(k >> 32)); }
__device__ __forceinline__ uint32_t desc_key_id(uint64_t k) { return (uint32_t)k; }

// ---------------------------------------------------------------- wave ops
// Lane exchange by a constant xor distance s, on the VALU instead of the LDS
// crossbar (ds_bpermute): DPP quad_perm for s = 1, 2; two DPP mirrors for s = 4;
// DPP row_ror:8 for s = 8; v_permlane16_swap / v_permlane32_swap for s = 16, 32.
// s must fold to a constant (it does inside fully unrolled loops).
__device__ __forceinline__ uint32_t lane_xor_u32(uint32_t v, int s) {
  const int lane = lane_id();
  switch (s) {
    case 1: return __builtin_amdgcn_update_dpp(0u, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    case 2: return __builtin_amdgcn_update_dpp(0u, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    case 4: {
      // row_half_mirror (l ^ 7 inside 8 lanes), then quad_perm [3,2,1,0] (l ^ 3): l ^ 4
      const int m = __builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false);
      return (uint32_t)__builtin_amdgcn_mov_dpp(m, 0x1B, 0xF, 0xF, false);
    }
    case 8: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false);   // row_ror:8 = l ^ 8
    case 16: {
      const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
      return (lane & 16) ? r[0] : r[1];
    }
    case 32: {
      const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
      return (lane & 32) ? r[0] : r[1];
    }
    default: return __shfl_xor(v, s);
  }
}
template <typename T> __device__ __forceinline__ T lane_xor(T v, int s) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "lane_xor: 32- or 64-bit values");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, lane_xor_u32(__builtin_bit_cast(uint32_t, v), s));
  } else {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = lane_xor_u32((uint32_t)u, s), hi = lane_xor_u32((uint32_t)(u >> 32), s);
    return __builtin_bit_cast(T, (hi << 32) | lo);
  }
}
// Start h0 and end h1 of sampled row `row`'s history in the id store: CSR offsets
// (off[row], off[row + 1]), a device-resident request slot s = slot[row] (ids
// s * cap .. s * cap + len[s]), or none (0, 0).  A slot outside [-1, nslots) or a length
// outside [0, cap] gives (0, -1), which every kernel treats as an invalid history.
// Where a row's sampled token goes: out_ids[row], and with device-resident histories that
// append in place, the end of the row's request slot (the next step's history,
// engine.py:242-246 with scheduler.py:281-284 appending each sampled id).  One thread per row
// calls put_id, once, where the row's token is final; a failed row (id -1) appends nothing,
// a full slot is counted in *overflow and not written.  Slot lengths are read by the row's
// own workgroups before that point and by no other row (the rows of a call name distinct
// slots).
struct IdSink {
  int64_t* out;
  const int32_t* slot;   // hist_slot, or NULL: no append
  int32_t* lens;
  int32_t* ids;
  int32_t* overflow;     // or NULL
  int32_t cap, nslots;
};
__device__ __forceinline__ void append_id(const IdSink& s, int row, int64_t id) {
  if (s.slot == nullptr || id < 0) return;
  const int32_t sl = s.slot[row];
  if (sl < 0 || sl >= s.nslots) return;
  const int32_t l = s.lens[sl];
  if (l >= 0 && l < s.cap) {
    s.ids[(int64_t)sl * s.cap + l] = (int32_t)id;
    s.lens[sl] = l + 1;
  } else if (s.overflow != nullptr) {
    atomicAdd(s.overflow, 1);
  }
}
__device__ __forceinline__ void put_id(const IdSink& s, int row, int64_t id) {
  s.out[row] = id;
  append_id(s, row, id);
}

__device__ __forceinline__ void row_history(const int32_t* off, const int32_t* slot, const int32_t* len,
                                            int32_t nslots, int32_t cap, int row, int32_t& h0, int32_t& h1) {
  h0 = 0;
  h1 = 0;
  if (off != nullptr) {
    h0 = off[row];
    h1 = off[row + 1];
  } else if (slot != nullptr) {
    const int32_t s = slot[row];
    if (s >= nslots || s < -1) {
      h1 = -1;
    } else if (s >= 0) {
      const int32_t n = len[s];
      h0 = s * cap;
      h1 = (n >= 0 && n <= cap) ? h0 + n : -1;
      if (h1 < 0) h0 = 0;
    }
  }
}
// A wave-uniform double taken from the first active lane (scalar registers).
__device__ __forceinline__ double uniform_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(u >> 32));
  return __builtin_bit_cast(double, (hi << 32) | lo);
}
// Value of lane `src` (wave-uniform) broadcast to every lane.
template <typename T> __device__ __forceinline__ T read_lane(T v, int src) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "read_lane: 32- or 64-bit values");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
  } else {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, src);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), src);
    return __builtin_bit_cast(T, (hi << 32) | lo);
  }
}
// DPP broadcast CTRL (0x142: lane 15 of each row to the next row; 0x143: lane 31 to rows 2 and
// 3) into the rows of RMASK; the other rows receive 0.
template <int CTRL, int RMASK, typename T> __device__ __forceinline__ T row_bcast_zero(T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "row_bcast_zero: 32- or 64-bit values");
  if constexpr (sizeof(T) == 4) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    return __builtin_bit_cast(T, (uint32_t)__builtin_amdgcn_update_dpp(0u, u, CTRL, RMASK, 0xF, false));
  } else {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0u, (uint32_t)u, CTRL, RMASK, 0xF, false);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0u, (uint32_t)(u >> 32), CTRL, RMASK, 0xF, false);
    return __builtin_bit_cast(T, (hi << 32) | lo);
  }
}
// Lane l receives lane l - s of its 16-lane row, or 0 where l - s leaves the row.
template <typename T> __device__ __forceinline__ T row_shr_zero(T v, int s) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "row_shr_zero: 32- or 64-bit values");
  if constexpr (sizeof(T) == 4) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    switch (s) {
      case 1: u = __builtin_amdgcn_update_dpp(0u, u, 0x111, 0xF, 0xF, true); break;
      case 2: u = __builtin_amdgcn_update_dpp(0u, u, 0x112, 0xF, 0xF, true); break;
      case 4: u = __builtin_amdgcn_update_dpp(0u, u, 0x114, 0xF, 0xF, true); break;
      default: u = __builtin_amdgcn_update_dpp(0u, u, 0x118, 0xF, 0xF, true); break;
    }
    return __builtin_bit_cast(T, u);
  } else {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = __builtin_bit_cast(uint32_t, row_shr_zero((uint32_t)u, s));
    const uint64_t hi = __builtin_bit_cast(uint32_t, row_shr_zero((uint32_t)(u >> 32), s));
    return __builtin_bit_cast(T, (hi << 32) | lo);
  }
}

template <typename T> __device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += lane_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_max_nan(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmax_nan(v, lane_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_min_nan(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmin_nan(v, lane_xor(v, o));
  return v;
}
template <typename T> __device__ __forceinline__ T wave_or(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v |= lane_xor(v, o);
  return v;
}
template <typename T> __device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) { T w = lane_xor(v, o); v = w > v ? w : v; }
  return v;
}
template <typename T> __device__ __forceinline__ T wave_min(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) { T w = lane_xor(v, o); v = w < v ? w : v; }
  return v;
}
// Inclusive prefix sum over the 64 lanes: Hillis-Steele inside each 16-lane
// row (DPP row_shr), then the three lower row totals added by readlane.
template <typename T> __device__ __forceinline__ T wave_incl_scan(T v) {
  // inside each row: lanes past the row's start read 0, so every lane adds unconditionally
  v += row_shr_zero(v, 1);
  v += row_shr_zero(v, 2);
  v += row_shr_zero(v, 4);
  v += row_shr_zero(v, 8);
  // across rows: row 1 and row 3 add the last lane of the row before them, then rows 2 and 3
  // add lane 31 (rows 0 and 1 together)
  v += row_bcast_zero<0x142, 0xA>(v);
  v += row_bcast_zero<0x143, 0xC>(v);
  return v;
}
__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// ---------------------------------------------------------- block helpers
// Scratch for cross-wave exchange: 16 waves x 4 doubles.
struct BlockScratch {
  double d[NWAVE][4];
};

__device__ __forceinline__ float block_max_nan(float v, BlockScratch* s) {
  v = wave_max_nan(v);
  if (lane_id() == 0) s->d[wave_id()][0] = (double)v;
  __syncthreads();
  float r = (float)s->d[0][0];
#pragma unroll
  for (int w = 1; w < NWAVE; ++w) r = fmax_nan(r, (float)s->d[w][0]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ float block_min_nan(float v, BlockScratch* s) {
  v = wave_min_nan(v);
  if (lane_id() == 0) s->d[wave_id()][0] = (double)v;
  __syncthreads();
  float r = (float)s->d[0][0];
#pragma unroll
  for (int w = 1; w < NWAVE; ++w) r = fmin_nan(r, (float)s->d[w][0]);
  __syncthreads();
  return r;
}
// Deterministic fixed-order sum (double).
__device__ __forceinline__ double block_sum(double v, BlockScratch* s) {
  v = wave_sum(v);
  if (lane_id() == 0) s->d[wave_id()][0] = v;
  __syncthreads();
  double r = 0.0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) r += s->d[w][0];
  __syncthreads();
  return r;
}
__device__ __forceinline__ int64_t block_sum_i64(int64_t v, BlockScratch* s) {
  v = wave_sum(v);
  if (lane_id() == 0) s->d[wave_id()][0] = __longlong_as_double(v);
  __syncthreads();
  int64_t r = 0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) r += __double_as_longlong(s->d[w][0]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ int64_t block_min_i64(int64_t v, BlockScratch* s) {
  v = wave_min(v);
  if (lane_id() == 0) s->d[wave_id()][0] = __longlong_as_double(v);
  __syncthreads();
  int64_t r = __double_as_longlong(s->d[0][0]);
#pragma unroll
  for (int w = 1; w < NWAVE; ++w) { int64_t x = __double_as_longlong(s->d[w][0]); r = x < r ? x : r; }
  __syncthreads();
  return r;
}
__device__ __forceinline__ int64_t block_max_i64(int64_t v, BlockScratch* s) {
  v = wave_max(v);
  if (lane_id() == 0) s->d[wave_id()][0] = __longlong_as_double(v);
  __syncthreads();
  int64_t r = __double_as_longlong(s->d[0][0]);
#pragma unroll
  for (int w = 1; w < NWAVE; ++w) { int64_t x = __double_as_longlong(s->d[w][0]); r = x > r ? x : r; }
  __syncthreads();
  return r;
}
// Whether any thread of the workgroup holds v (one word per wave; two barriers).
__device__ __forceinline__ bool block_any(bool v, BlockScratch* s) {
  int32_t* words = reinterpret_cast<int32_t*>(s);
  const bool w = ballot(v) != 0ull;
  if (lane_id() == 0) words[wave_id()] = w ? 1 : 0;
  __syncthreads();
  const int l = lane_id();
  const bool r = ballot(l < NWAVE && words[l < NWAVE ? l : 0] != 0) != 0ull;
  __syncthreads();
  return r;
}
// Exclusive prefix over threads in thread order (double); *total receives the block sum.
__device__ __forceinline__ double block_excl_scan(double v, double* total, BlockScratch* s) {
  double inc = wave_incl_scan(v);
  if (lane_id() == 63) s->d[wave_id()][1] = inc;
  __syncthreads();
  double off = 0.0, tot = 0.0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    double t = s->d[w][1];
    if (w < wave_id()) off += t;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return off + inc - v;
}
__device__ __forceinline__ int block_excl_scan_int(int v, int* total, BlockScratch* s) {
  int inc = wave_incl_scan(v);
  if (lane_id() == 63) s->d[wave_id()][1] = (double)inc;
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    int t = (int)s->d[w][1];
    if (w < wave_id()) off += t;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return off + inc - v;
}

// ------------------------------------------------------- buffer loads
// Raw buffer loads through a resource descriptor: the base address lives in
// scalar registers and one 32-bit offset register serves every load of a thread;
// loads at or past `nbytes` return zeros (hardware range check).  Word 3 of the
// descriptor is the gfx9-family value for untyped dword access.
typedef unsigned int ns_v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const ns_v4u x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
  return make_uint4(x.x, x.y, x.z, x.w);
}
// The same load with the non-temporal cache policy (aux bit 1): a streaming read of data
// the kernel does not read again from the caches; measured 0.8 us faster than the default
// policy over a 65.7 MB decode batch of rows on MI355X.
__device__ __forceinline__ uint4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  const ns_v4u x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, 2);
  return make_uint4(x.x, x.y, x.z, x.w);
}
// 16 bytes at byte off + voff of a region of nbytes bytes (both multiples of 16).  One
// descriptor over the region, the whole offset in the VGPR operand, which the range
// check covers: loads past the region read zero and touch no memory.  (A descriptor
// per offset would be computed in VGPRs and turn every load into a waterfall loop.)
__device__ __forceinline__ uint4 buf_load16_at(const unsigned char* base, uint32_t nbytes, uint32_t off,
                                               uint32_t voff) {
  return buf_load16(make_rsrc(base, nbytes), voff + off, 0u);
}

// exp from the ROCm device library (ocml expf, faithfully rounded); not the
// reduced-precision __expf.
__device__ __forceinline__ float ns_expf(float x) { return expf(x); }

// 1/x in float64 for a positive normal x: the hardware reciprocal estimate refined by two
// Newton-Raphson steps (r' = r + r * (1 - x * r)), a few units in the last place of the
// correctly rounded quotient, without the scaling and fix-up sequence of IEEE division.
__device__ __forceinline__ double rcp_f64(double x) {
  double r = __builtin_amdgcn_rcp(x);
  double e = __builtin_fma(-x, r, 1.0);
  r = __builtin_fma(r, e, r);
  e = __builtin_fma(-x, r, 1.0);
  return __builtin_fma(r, e, r);
}

// ------------------------------------------------- exact division x / t
// Correctly rounded quotient by a row-uniform divisor t > 0 with precomputed
// r = RN(1/t): q0 = RN(x*r); rem = fma(-q0, t, x) is exact; q = RN(q0 + rem*r)
// (Markstein's correction theorem for a correctly rounded reciprocal).  The theorem's
// conditions: r normal and correctly rounded (t in [2^-100, 2^100]), q0 and q normal
// (|q0| in [2^-100, 2^100]), and rem exact, which holds when it is a multiple of the
// smallest subnormal: rem is a multiple of ulp(q0) * ulp(t), at least |x| * 2^-48, so
// |x| >= 2^-100 suffices; |q0| >= 2^-99 * r gives that.  div_lo(t, r) folds these into
// one lower bound on |q0| (+inf: never), computed once per divisor; outside it the IEEE
// division is used.  Bit-exactness against IEEE x/t is tested on the CPU over every
// binade of the float range for a set of divisors.
__host__ __device__ __forceinline__ float div_lo(float t, float r) {
  return (t >= 0x1.0p-100f && t <= 0x1.0p+100f) ? __builtin_fmaxf(0x1.0p-100f, 0x1.0p-99f * r)
                                                 : __builtin_inff();
}
__device__ __forceinline__ float div_rn(float x, float t, float r) {
  float q0 = x * r;
  float rem = __builtin_fmaf(-q0, t, x);
  float q = __builtin_fmaf(rem, r, q0);
  float aq = __builtin_fabsf(q0);
  bool slow = !(aq >= div_lo(t, r) && aq <= 0x1.0p+100f);
  if (__ballot(slow) != 0ull) {  // wave-uniform branch: the IEEE division is never speculated
    asm volatile("");             // (the empty asm keeps the compiler from if-converting it)
    if (slow) q = x / t;
  }
  return q;
}

// The NaN guard's uniform row (sampler.py:77-80).  Every token's probability is the float32
// 1/V: RN32(1/V) equals RN32(RN64(1/V)) for every V up to 2^18 (every one checked on the CPU),
// so the float32 division gives torch's value.  The pick is the i with i * q <= u < (i + 1) * q
// in float64 (exact: i < 2^18 times a 24-bit q), V - 1 if none; the loops reach it from any
// start, and u * V is within one step of it.
__device__ __forceinline__ float uniform_q(int64_t V) { return 1.0f / (float)V; }
__device__ __forceinline__ int64_t uniform_pick(float u, float q, int64_t V) {
  const double qd = q, ud = u;
  int64_t i = (int64_t)(ud * (double)V);
  while (i > 0 && (double)i * qd > ud) --i;
  while ((double)(i + 1) * qd <= ud && i < V) ++i;
  return i >= V ? V - 1 : i;
}

// The arrival ticket of a row split over several workgroups, taken by one thread of each after
// its workgroup's hand-over data is stored and a barrier.  Returns true in the last arrival.
// The hand-over needs no release/acquire fence pair: every datum crosses workgroups through
// agent-scope atomic stores and loads, which gfx950 serves at the device coherence point
// (they bypass the per-XCD L2s), and each wave's s_waitcnt vmcnt(0) before the barrier
// completes its stores there before the counter moves.  An agent-scope release / acquire
// (buffer_wbl2 / buffer_inv of the whole L2) measured 27% to 59% slower on the split-row
// paths.  A launch cut short leaves its counters nonzero: the caller then clears the buffer
// that holds them before the next call.
__device__ __forceinline__ bool arrive_last(int32_t* counter, int32_t arrivals) {
  return atomicAdd(counter, 1) == arrivals - 1;
}

// The repetition penalty of one history token (sampler.py:37: score * p if score < 0 else
// score / p), float32; rpen = RN(1/pen).  recip = false: the division correctly rounded (torch
// on the CPU); recip = true: x * rpen (torch on a GPU divides a tensor by a Python float that
// way).  recip is the same for every lane of a launch.
__device__ __forceinline__ float pen_rn(float x, float pen, float rpen, bool recip) {
  return x < 0.0f ? x * pen : (recip ? x * rpen : div_rn(x, pen, rpen));
}

}  // namespace ns
