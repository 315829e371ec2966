// Device-side building blocks for the gfx950 flash-spacetime kernels.
//
// Conventions. A wavefront is 64 lanes; lane = 16*g + n with lane group
// g in 0..3 and n in 0..15. The MFMA tiles used are 16x16 with the layouts
// measured on gfx950:
//   A (M x K): lane (g, n) holds A[m = n][k-slots of group g]
//   B (K x N): lane (g, n) holds B[k-slots of group g][n = n]
//   C (M x N): lane (g, n) holds C[m = 4g + r][n], r = 0..3 (one f32x4)
// k-slots of group g: bf16 16x16x32 -> k = 8g .. 8g+7, bf16 16x16x16 ->
// k = 4g .. 4g+3, fp32 16x16x4 -> k = g. Consecutive MFMAs that accumulate
// into one register quad always use the same opcode (see KFrag<bf16, K>).
//
// Two operand families are used:
//  * KFrag<T, K>: contraction over a contiguous feature axis of length K
//    (head dim D or channel count C), slots as above, loaded straight from
//    memory where that axis is innermost.
//  * JFrag<T, NS>: contraction over a chunk of NS 16-key subtiles. Slot t
//    of group g is key 16*(t/4) + 4g + (t%4), which is exactly how the C
//    tiles of the subtiles lay keys out, so a probability tile computed as
//    S^T = K Q^T is consumed by the next MFMA without any data movement.
//    fp32 uses 4*NS 16x16x4 steps; step t = 4s + r holds key 16s + 4g + r.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fst {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Spec constants (reference.py:39-42); 3e4/500*3e-1 == 18 exactly.
constexpr float kTimeScale = 18.0f;
constexpr float kInputScale = 1024.0f;
constexpr float kClip = 4.0f;

template <typename T>
struct is_bf16 {
  static constexpr bool value = false;
};
template <>
struct is_bf16<bf16> {
  static constexpr bool value = true;
};

__device__ __forceinline__ f32x4 mfma_x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_x16(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// fp32 quad -> bf16 quad (round to nearest even) as two v_cvt_pk_bf16_f32.
// Converted pairwise through 32-bit words: converting the quad directly is
// split into single conversions plus permutes by the instruction selector
// when the result feeds an MFMA operand.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ bf16x4 pack4(const f32x4& c) {
  const unsigned lo = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{c[0], c[1]}, bf16x2));
  const unsigned hi = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{c[2], c[3]}, bf16x2));
  return __builtin_bit_cast(bf16x4, u32x2v{lo, hi});
}

// ---------------------------------------------------------------------------
// Cross-lane reductions over the four lane groups (lanes n, n+16, n+32,
// n+48) with the gfx950 row-swap instructions; every lane ends with the
// result.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float group_allmax(float x) {
  unsigned u = __float_as_uint(x);
  auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  unsigned w = __float_as_uint(y);
  auto b = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float group_allsum(float x) {
  unsigned u = __float_as_uint(x);
  auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  unsigned w = __float_as_uint(y);
  auto b = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Two sums at once, with the additions of group_allsum in the same order:
// the first swap gives lanes 0-31 the half sums of x and lanes 32-63 those of
// y, the second completes both, and a last swap hands each value to every
// lane (three swaps where two group_allsum calls take four and two copies).
__device__ __forceinline__ void group_allsum2(float& x, float& y) {
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  const float c = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const unsigned uc = __float_as_uint(c);
  auto b = __builtin_amdgcn_permlane16_swap(uc, uc, false, false);
  const float e = __uint_as_float(b[0]) + __uint_as_float(b[1]);
  const unsigned ue = __float_as_uint(e);
  auto d = __builtin_amdgcn_permlane32_swap(ue, ue, false, false);
  x = __uint_as_float(d[0]);
  y = __uint_as_float(d[1]);
}

// Orders this wave's LDS accesses: everything issued before completes
// before anything after is issued (LDS executes a wave's requests in order).
__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// ---------------------------------------------------------------------------
// Feature-axis operands.
// ---------------------------------------------------------------------------
template <typename T, int K>
struct KFrag;

template <int K>
struct KFrag<bf16, K> {
  // Axes that are a multiple of 32 contract with 16x16x32 steps (slots
  // k = 32t + 8g .. +7); others (16, 48) with 16x16x16 steps only (slots
  // k = 16t + 4g .. +3). The two step kinds are never chained on one
  // accumulator: hipcc for gfx950 emits a 16x16x32 -> 16x16x16 SrcC chain
  // without the wait states it needs, which gave wrong and run-to-run
  // different results.
  static_assert(K % 16 == 0, "bf16 feature axis must be a multiple of 16");
  static constexpr int N32 = (K % 32 == 0) ? K / 32 : 0;
  static constexpr int N16 = (K % 32 == 0) ? 0 : K / 16;
  bf16x8 x32[N32 > 0 ? N32 : 1];
  bf16x4 x16[N16 > 0 ? N16 : 1];

  // Zero unless ok, without a branch (selects on the 32-bit words).
  __device__ __forceinline__ void keep_if(bool ok) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int t = 0; t < N32; ++t) {
      const u32x4 v = __builtin_bit_cast(u32x4, x32[t]);
      x32[t] = __builtin_bit_cast(bf16x8, ok ? v : u32x4{0u, 0u, 0u, 0u});
    }
#pragma unroll
    for (int t = 0; t < N16; ++t) {
      const u32x2 v = __builtin_bit_cast(u32x2, x16[t]);
      x16[t] = __builtin_bit_cast(bf16x4, ok ? v : u32x2{0u, 0u});
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int t = 0; t < N32; ++t)
#pragma unroll
      for (int e = 0; e < 8; ++e) x32[t][e] = (bf16)0.f;
#pragma unroll
    for (int t = 0; t < N16; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) x16[t][e] = (bf16)0.f;
  }
  // p points at element 0 of this lane's row (16-byte aligned rows).
  __device__ __forceinline__ void load(const bf16* p, int g) {
#pragma unroll
    for (int t = 0; t < N32; ++t) x32[t] = *reinterpret_cast<const bf16x8*>(p + 32 * t + 8 * g);
#pragma unroll
    for (int t = 0; t < N16; ++t) x16[t] = *reinterpret_cast<const bf16x4*>(p + 16 * t + 4 * g);
  }
  // The inverse of load: this lane's slots back to element 0 of its row.
  __device__ __forceinline__ void store(bf16* p, int g) const {
#pragma unroll
    for (int t = 0; t < N32; ++t) *reinterpret_cast<bf16x8*>(p + 32 * t + 8 * g) = x32[t];
#pragma unroll
    for (int t = 0; t < N16; ++t) *reinterpret_cast<bf16x4*>(p + 16 * t + 4 * g) = x16[t];
  }
  // bf16(float(x) * scale): the reference's q * scale before the cast.
  __device__ __forceinline__ void scale_by(float scale) {
#pragma unroll
    for (int t = 0; t < N32; ++t)
#pragma unroll
      for (int e = 0; e < 8; ++e) x32[t][e] = (bf16)((float)x32[t][e] * scale);
#pragma unroll
    for (int t = 0; t < N16; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) x16[t][e] = (bf16)((float)x16[t][e] * scale);
  }
  __device__ __forceinline__ void load_scaled(const bf16* p, int g, float scale) {
    load(p, g);
    scale_by(scale);
  }
  // Per-lane feature slots (as dot_minus_slots takes them): N32 groups of
  // 8 (features 32t + 8g ..), then N16 groups of 4 (features 16t + 4g ..).
  static constexpr int SLOTS = N32 * 8 + N16 * 4;
  // This lane's part of sum_k x_k (o_k - b_k) over the row, b in slots.
  __device__ __forceinline__ float dot_minus_slots(const KFrag& o, const float* bs) const {
    float a = 0.f;
#pragma unroll
    for (int t = 0; t < N32; ++t)
#pragma unroll
      for (int e = 0; e < 8; ++e) a = __builtin_fmaf((float)x32[t][e], (float)o.x32[t][e] - bs[8 * t + e], a);
#pragma unroll
    for (int t = 0; t < N16; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        a = __builtin_fmaf((float)x16[t][e], (float)o.x16[t][e] - bs[N32 * 8 + 4 * t + e], a);
    return a;
  }
};

template <int K>
struct KFrag<float, K> {
  // fp32 16x16x4: step t, lane group g holds k = (K/4) g + t, so a lane's
  // operand is one contiguous quarter of the row.
  static_assert(K % 16 == 0, "fp32 feature axis must be a multiple of 16");
  static constexpr int Q = K / 4;
  float x[Q];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int t = 0; t < Q; ++t) x[t] = 0.f;
  }
  __device__ __forceinline__ void load(const float* p, int g) {
#pragma unroll
    for (int t = 0; t < Q; t += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(p + Q * g + t);
      x[t] = v[0]; x[t + 1] = v[1]; x[t + 2] = v[2]; x[t + 3] = v[3];
    }
  }
  __device__ __forceinline__ void load_scaled(const float* p, int g, float scale) {
    load(p, g);
#pragma unroll
    for (int t = 0; t < Q; ++t) x[t] *= scale;
  }
};

template <int K>
__device__ __forceinline__ f32x4 mma_k(const KFrag<bf16, K>& a, const KFrag<bf16, K>& b, f32x4 c) {
#pragma unroll
  for (int t = 0; t < KFrag<bf16, K>::N32; ++t) c = mfma_x32(a.x32[t], b.x32[t], c);
#pragma unroll
  for (int t = 0; t < KFrag<bf16, K>::N16; ++t) c = mfma_x16(a.x16[t], b.x16[t], c);
  return c;
}

template <int K>
__device__ __forceinline__ f32x4 mma_k(const KFrag<float, K>& a, const KFrag<float, K>& b, f32x4 c) {
#pragma unroll
  for (int t = 0; t < K / 4; ++t) c = mfma_f32(a.x[t], b.x[t], c);
  return c;
}

// ---------------------------------------------------------------------------
// Key-chunk operands: NS 16-key subtiles (chunk of 16*NS keys).
// ---------------------------------------------------------------------------
template <typename T, int NS>
struct JFrag;

// bf16, 32 keys: one 16x16x32 step.
template <>
struct JFrag<bf16, 2> {
  bf16x8 v;
  __device__ __forceinline__ void from_tiles(const f32x4* s) {
    v = __builtin_shufflevector(pack4(s[0]), pack4(s[1]), 0, 1, 2, 3, 4, 5, 6, 7);
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = (bf16)0.f;
  }
  // Keys contiguous in memory (p -> key 0 of this lane's key row).
  __device__ __forceinline__ void load_keys(const bf16* p, int g) {
    const bf16x4 lo = *reinterpret_cast<const bf16x4*>(p + 4 * g);
    const bf16x4 hi = *reinterpret_cast<const bf16x4*>(p + 16 + 4 * g);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      v[r] = lo[r];
      v[4 + r] = hi[r];
    }
  }
  __device__ __forceinline__ void store_keys(bf16* p, int g) const {
    bf16x4 lo, hi;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      lo[r] = v[r];
      hi[r] = v[4 + r];
    }
    *reinterpret_cast<bf16x4*>(p + 4 * g) = lo;
    *reinterpret_cast<bf16x4*>(p + 16 + 4 * g) = hi;
  }
  // Keys along the rows of an LDS matrix whose innermost axis is the free
  // index (base -> [key 0][col 0]); lane (g, n) receives M[key][col0 + n]
  // through transposing reads (within a 16-lane group, slot t of lane n comes
  // from the address given by lane 4t + n/4, element n%4).
  __device__ __forceinline__ void load_tr(const bf16* base, int row_stride, int col0, int g, int n) {
    const bf16* p = base + (4 * g + (n >> 2)) * row_stride + col0 + 4 * (n & 3);
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p + 16 * row_stride));
    v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  }
};

// bf16, 16 keys: one 16x16x16 step.
template <>
struct JFrag<bf16, 1> {
  bf16x4 v;
  __device__ __forceinline__ void from_tiles(const f32x4* s) { v = pack4(s[0]); }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int t = 0; t < 4; ++t) v[t] = (bf16)0.f;
  }
  __device__ __forceinline__ void load_keys(const bf16* p, int g) { v = *reinterpret_cast<const bf16x4*>(p + 4 * g); }
  __device__ __forceinline__ void store_keys(bf16* p, int g) const { *reinterpret_cast<bf16x4*>(p + 4 * g) = v; }
  __device__ __forceinline__ void load_tr(const bf16* base, int row_stride, int col0, int g, int n) {
    const bf16* p = base + (4 * g + (n >> 2)) * row_stride + col0 + 4 * (n & 3);
    v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
  }
};

// fp32: 4*NS 16x16x4 steps; step 4s + r holds key 16s + 4g + r.
template <int NS>
struct JFrag<float, NS> {
  float v[4 * NS];
  __device__ __forceinline__ void from_tiles(const f32x4* s) {
#pragma unroll
    for (int q = 0; q < NS; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) v[4 * q + r] = s[q][r];
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int t = 0; t < 4 * NS; ++t) v[t] = 0.f;
  }
  __device__ __forceinline__ void load_keys(const float* p, int g) {
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(p + 16 * q + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) v[4 * q + r] = a[r];
    }
  }
  __device__ __forceinline__ void store_keys(float* p, int g) const {
#pragma unroll
    for (int q = 0; q < NS; ++q)
      *reinterpret_cast<f32x4*>(p + 16 * q + 4 * g) = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
  }
  __device__ __forceinline__ void load_tr(const float* base, int row_stride, int col0, int g, int n) {
#pragma unroll
    for (int q = 0; q < NS; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) v[4 * q + r] = base[(16 * q + 4 * g + r) * row_stride + col0 + n];
  }
};

__device__ __forceinline__ f32x4 mma_j(const JFrag<bf16, 2>& a, const JFrag<bf16, 2>& b, f32x4 c) {
  return mfma_x32(a.v, b.v, c);
}
__device__ __forceinline__ f32x4 mma_j(const JFrag<bf16, 1>& a, const JFrag<bf16, 1>& b, f32x4 c) {
  return mfma_x16(a.v, b.v, c);
}
template <int NS>
__device__ __forceinline__ f32x4 mma_j(const JFrag<float, NS>& a, const JFrag<float, NS>& b, f32x4 c) {
#pragma unroll
  for (int t = 0; t < 4 * NS; ++t) c = mfma_f32(a.v[t], b.v[t], c);
  return c;
}

// ---------------------------------------------------------------------------
// Pair geometry (reference.py:75-84, _tiles.py:25-60).
// ---------------------------------------------------------------------------

// x_ij = 1024 * clip(sign(I) sqrt|I|, -4, 4), I = |dp|^2 - (18 dt)^2, fp32.
__device__ __forceinline__ float pair_angle(float4 a, float4 b) {
  float dx = a.x - b.x, dy = a.y - b.y, dz = a.z - b.z;
  float dt = (a.w - b.w) * kTimeScale;
  float interval = __builtin_fmaf(dx, dx, __builtin_fmaf(dy, dy, __builtin_fmaf(dz, dz, -dt * dt)));
  float mag = __builtin_amdgcn_sqrtf(fabsf(interval));
  float sd = interval > 0.f ? mag : (interval < 0.f ? -mag : 0.f);
  return kInputScale * fminf(fmaxf(sd, -kClip), kClip);
}

// The same angle evaluated in binary64 from the fp32 coordinates (the
// differences are exact there, so only the final rounding remains). Used by
// the fp32 kernels: near the light cone I is a difference of nearly equal
// squares, and any fp32 evaluation of it carries an error that is large
// relative to I; in binary64 that error is gone, so the fp32 kernels are at
// least as accurate as the eager fp32 definition on every pair.
__device__ __forceinline__ double pair_angle_f64(float4 a, float4 b) {
  const double dx = (double)a.x - (double)b.x, dy = (double)a.y - (double)b.y, dz = (double)a.z - (double)b.z;
  const double dt = ((double)a.w - (double)b.w) * 18.0;
  const double interval = dx * dx + dy * dy + dz * dz - dt * dt;
  const double mag = __builtin_sqrt(__builtin_fabs(interval));
  const double sd = interval > 0.0 ? mag : (interval < 0.0 ? -mag : 0.0);
  return 1024.0 * __builtin_fmin(__builtin_fmax(sd, -4.0), 4.0);
}

// Frequency table handed to the kernels: ghi + glo = f_c / (2 pi) split in
// two fp32 words (the hardware sin/cos take revolutions), and whether the
// largest angle 4096 f_c exceeds the +-256 revolution domain of v_sin_f32,
// in which case the argument is reduced with v_fract_f32 first.
struct FreqTable {
  float ghi[32];
  float glo[32];
  uint32_t reduce_mask;  // bit f set -> reduce channel pair f
};

// sin and cos of 2*pi*(x * g) for one frequency. ACCURATE (fp32 embedding)
// reduces to [0, 1) revolutions and adds the low word of g and the rounding
// error of x*ghi (two FMAs), so the argument is good to ~1e-7 revolutions
// even at |x*g| ~ 650; otherwise (bf16 embedding) only arguments beyond the
// +-256 revolution domain are reduced and the argument carries the fp32
// rounding of the product (<= 1.5e-5 rev), far below the bf16 rounding the
// embedding gets next.
template <bool ACCURATE>
__device__ __forceinline__ void sincos_rev(float x, float ghi, float glo, bool reduce, float& s, float& c) {
  float p = x * ghi;
  float r;
  if constexpr (ACCURATE) {
    // Every channel is reduced to [0, 1) before the correction is added, so
    // the correction is not lost to the ulp of a large argument.
    float e = __builtin_fmaf(x, ghi, -p);
    e = __builtin_fmaf(x, glo, e);
    r = __builtin_amdgcn_fractf(p) + e;
  } else {
    r = reduce ? __builtin_amdgcn_fractf(p) : p;
  }
  s = __builtin_amdgcn_sinf(r);
  c = __builtin_amdgcn_cosf(r);
}

}  // namespace fst
