// Shared kernel parameters and helpers of the flash-spacetime HIP library.
#pragma once

#include "fst_device.h"
#include "../../include/flash_spacetime.h"

namespace fst {

// Event layout shared by every kernel: padded [B, H, L, X] with seqlens, or
// packed [T, H, X] with cu_seqlens (forward.py:247-255, _tiles.py:80-117).
// Padded events may also be stored token-major, [B, L, H, X] (vectors
// [B, L, H]): the layout a [B, L, H*D] projection has before its heads are
// split, so the heads-first views a model passes are read in place.
struct EventSpec {
  const int32_t* lens;    // seqlens [B] (padded) or the work list's sanitised cu_seqlens [B+1] (packed)
  const int32_t* blkcum;  // [B+1] prefix sums of row blocks per event
  const int32_t* perm;    // [B] events by decreasing length (the tile kernels' schedules)
  const int32_t* scum;    // [B+1] packed: prefix sums of row blocks in perm order (or null)
  // [8 ceil(B / 8) + 1] padded: prefix sums of the valid (not padding-only)
  // 16-row tiles over the events in XCD order (entry x S + j: XCD x's j-th
  // event, S = ceil(B / 8)), for tile_block's padding-last schedule; or null.
  const int32_t* vp;
  const float4* pos4;     // [B*L] or [T] (x, y, z, t) fp32
  const int32_t* status;  // the work list's verdict on the call's lengths: 0 = well formed (or null)
  int B, H, L, T, packed;
  int tokmajor;           // rows of one token's heads are adjacent (packed, or padded token-major)
  int xmul;               // 3: q, k, v (and dq, dk, dv) interleaved per token as [.., 3, H, X]; else 1
  int max_len;            // longest event whose rows of all heads span less than 2^31 bytes
};

struct EventBlock {
  int b, blk, len, tok0;
};

// Row addressing of one event. Offsets are in elements of a row of width X.
struct RowAddr {
  long base_row;  // row index of (token 0, head 0)
  long hs, ts;    // row strides of head and token
  long pos_base;
  __device__ __forceinline__ long vec(int h, int i) const { return base_row + h * hs + i * ts; }
  __device__ __forceinline__ long off(int h, int i, int width) const { return vec(h, i) * width; }
  __device__ __forceinline__ float4 pos(const float4* p4, int i) const { return p4[pos_base + i]; }
};

// Token range of event b, clamped into the tensor: padded lengths to [0, L],
// packed offsets to [0, T] and non-decreasing. The packed offsets the
// kernels read are the work list's sanitised copy (running maximum of the
// caller's offsets, clamped to [0, T]), so events never overlap and their
// row blocks never outnumber the per-tile slots sized from T.
__device__ __forceinline__ void event_range(const EventSpec& ev, int b, int& tok0, int& len) {
  if (ev.packed) {
    int a = ev.lens[b], e = ev.lens[b + 1];
    a = a < 0 ? 0 : (a > ev.T ? ev.T : a);
    e = e < a ? a : (e > ev.T ? ev.T : e);
    tok0 = a;
    len = e - a;
  } else {
    const int l = ev.lens[b];
    tok0 = 0;
    len = l < 0 ? 0 : (l > ev.L ? ev.L : l);
  }
}

// Whether the kernels refuse event eb and write NaN into its rows instead of
// computing: the call's packed offsets were malformed (the work list found
// cu_seqlens[0] != 0, a decreasing offset, or cu_seqlens[B] > T, and ran on
// sanitised offsets so that no access leaves the tensors), or the event's
// rows of all heads span 2^31 bytes or more, past the 32-bit byte offsets of
// the buffer loads (which would read zeros there).
__device__ __forceinline__ bool event_refused(const EventSpec& ev, const EventBlock& eb) {
  return (ev.status && *ev.status != 0) || eb.len > ev.max_len;
}

// NaN into rows [r0, r1) of every head of a refused event: out (rows of
// width X, addressed by ra) and vec (per-row scalars addressed by rv, when
// not null).
template <typename T, int X>
__device__ void fill_rows_nan(const RowAddr& ra, const RowAddr& rv, int r0, int r1, int H, int tid, int nthreads,
                              T* out, float* vec) {
  if (r1 <= r0) return;
  const int nr = r1 - r0;
  for (int idx = tid; idx < H * nr * X; idx += nthreads) {
    const int c = idx % X, r = (idx / X) % nr, h = idx / (X * nr);
    out[ra.off(h, r0 + r, X) + c] = (T)__builtin_nanf("");
  }
  if (vec)
    for (int idx = tid; idx < H * nr; idx += nthreads) vec[rv.vec(idx / nr, r0 + idx % nr)] = __builtin_nanf("");
}

// Largest i in [0, n) with key(i) <= t, for key nondecreasing in i and
// key(0) <= t. Each round the wave reads 64 evenly spaced entries of the
// range left (one load per lane) and the count of those at or below t
// (a ballot) narrows it to one gap: one round for n <= 64, two for n <= 4096,
// where a binary search would chain log2 n dependent loads. The result is
// the same in every lane of the wave.
template <typename F>
__device__ __forceinline__ int wave_last_le(int n, int t, F key) {
  const int lane = threadIdx.x & 63;
  int lo = 0, len = n;
  while (len > 1) {
    const int step = (len + 63) >> 6;
    const int i = lo + lane * step;
    const bool le = i < lo + len && key(i) <= t;
    const int c = __builtin_popcountll(__builtin_amdgcn_ballot_w64(le));
    const int nlo = lo + (c - 1) * step;
    len = min(step, lo + len - nlo);
    lo = nlo;
  }
  return __builtin_amdgcn_readfirstlane(lo);
}

// Work item of workgroup w: the event whose blocks hold w (blkcum[0] == 0).
__device__ __forceinline__ bool locate_block(const EventSpec& ev, int w, EventBlock& eb) {
  if (w >= ev.blkcum[ev.B]) return false;
  const int32_t* bc = ev.blkcum;
  const int lo = wave_last_le(ev.B, w, [&](int i) { return bc[i]; });
  eb.b = lo;
  eb.blk = w - ev.blkcum[lo];
  event_range(ev, lo, eb.tok0, eb.len);
  return true;
}

__device__ __forceinline__ RowAddr row_addr(const EventSpec& ev, const EventBlock& eb) {
  RowAddr r;
  if (ev.packed) {
    r.base_row = (long)eb.tok0 * ev.H;
    r.hs = 1;
    r.ts = ev.H;
    r.pos_base = eb.tok0;
  } else if (ev.tokmajor) {
    r.base_row = (long)eb.b * ev.L * ev.H;
    r.hs = 1;
    r.ts = ev.H;
    r.pos_base = (long)eb.b * ev.L;
  } else {
    r.base_row = (long)eb.b * ev.H * ev.L;
    r.hs = ev.L;
    r.ts = 1;
    r.pos_base = (long)eb.b * ev.L;
  }
  return r;
}

// Register load of a four-wave bf16 rows-kernel lane, in the units of
// (HP / 4) D + 3 C: at 160 and more such instances spill, and the rows kernel
// runs eight waves instead (which needs HP % 8 == 0).
__host__ __device__ constexpr int rows_wave_load(int HP, int D, int C) { return (HP / 4) * D + 3 * C; }

// Row addressing of q, k, v, dq, dk and dv. With the operands interleaved
// per token (one [.., 3, H, D] projection output), a token's q heads are
// followed by its k heads and v heads: the token stride is three times that
// of out, grad_out and the per-row vectors, and k, v start H D elements
// after q.
__device__ __forceinline__ RowAddr row_addr_x(const EventSpec& ev, const EventBlock& eb) {
  RowAddr r = row_addr(ev, eb);
  if (ev.xmul > 1) {
    r.base_row *= ev.xmul;
    r.ts *= ev.xmul;
  }
  return r;
}

struct FwdParams {
  EventSpec ev;
  int H, flags;
  float scale;
  const void *q, *k, *v;
  const float* weight;  // [D, C]
  const float* bias;    // [D] or null
  void* out;
  float* lse;
  FreqTable freq;
};

struct BwdParams {
  EventSpec ev;     // rows-kernel work list in ev.blkcum
  const int32_t* blkcum_cols;  // cols-kernel work list
  const int32_t* scum_cols;    // its packed schedule (row blocks in ev.perm order), or null
  int H, flags;
  float scale;
  const void *q, *k, *v, *dout;
  const float* weight;  // [D, C]
  const float* bias;    // [D] or null
  const float* lse;     // [rows]
  const void* out;      // the forward's output, laid out as dout (nullable; bf16 rows kernel)
  // scratch written by the rows kernel, read by the cols kernel
  void* u;              // [rows, C] T
  void* wt;             // [rows, C] T
  void* qt;             // [rows, D] T: bf16(q * scale) (written by the bf16 rows kernel)
  float* dob;           // [rows]
  float* dsum;          // [rows]
  // [rows] the rows kernel's sum of P per row, Z, for the cols kernel's P / Z:
  // bf16, the log2-domain LSE of the normalised P, lse log2(e) + log2 Z;
  // float32, log2 Z alone (at logits of O(1e4) the sum would round away the
  // correction, so the float32 cols kernel subtracts it after the exponent's
  // fma).
  float* lse_z;
  float* dw_part;       // [blocks, D, C]
  float* db_part;       // [blocks, D]
  // outputs
  void *dq, *dk, *dv;
  float* rowsum;        // nullable
  float* dweight;
  float* dbias;         // nullable
  FreqTable freq;
};

template <typename T>
struct VecOf;
template <>
struct VecOf<bf16> {
  typedef bf16x8 type;
  static __device__ __forceinline__ bf16x8 zero() {
    bf16x8 z;
#pragma unroll
    for (int e = 0; e < 8; ++e) z[e] = (bf16)0.f;
    return z;
  }
};
template <>
struct VecOf<float> {
  typedef f32x4 type;
  static __device__ __forceinline__ f32x4 zero() { return zero4(); }
};

__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Completion of this wave's outstanding buffer loads (including loads into
// LDS), ordered against every later memory access of the wave.
__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Four consecutive output elements from an fp32 quad.
template <typename T>
__device__ __forceinline__ void store4(T* p, const f32x4& v);
template <>
__device__ __forceinline__ void store4<bf16>(bf16* p, const f32x4& v) {
  bf16x4 o;
#pragma unroll
  for (int r = 0; r < 4; ++r) o[r] = (bf16)v[r];
  *reinterpret_cast<bf16x4*>(p) = o;
}
template <>
__device__ __forceinline__ void store4<float>(float* p, const f32x4& v) {
  *reinterpret_cast<f32x4*>(p) = v;
}

// ---------------------------------------------------------------------------
// Channel operand of the u.E / w~.E contractions (K = C). Slot r of lane
// group g in channel tile ct is channel 16ct + 4g + r -- the C layout of a
// 16x16 fp32 MFMA tile -- so U computed on the MFMA feeds the next one
// directly. bf16 contracts each tile with one 16x16x16 step; fp32 with four
// 16x16x4 steps (step r covers channels 16ct + r + {0, 4, 8, 12}).
// ---------------------------------------------------------------------------
template <typename T, int C>
struct CFrag;

template <int C>
struct CFrag<bf16, C> {
  bf16x4 v[C / 16];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int ct = 0; ct < C / 16; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) v[ct][r] = (bf16)0.f;
  }
  __device__ __forceinline__ void load(const bf16* p, int g) {
#pragma unroll
    for (int ct = 0; ct < C / 16; ++ct) v[ct] = *reinterpret_cast<const bf16x4*>(p + 16 * ct + 4 * g);
  }
  __device__ __forceinline__ void from_acc(const f32x4* acc) {
#pragma unroll
    for (int ct = 0; ct < C / 16; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) v[ct][r] = (bf16)acc[ct][r];
  }
};

template <int C>
struct CFrag<float, C> {
  f32x4 v[C / 16];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int ct = 0; ct < C / 16; ++ct) v[ct] = zero4();
  }
  __device__ __forceinline__ void load(const float* p, int g) {
#pragma unroll
    for (int ct = 0; ct < C / 16; ++ct) v[ct] = *reinterpret_cast<const f32x4*>(p + 16 * ct + 4 * g);
  }
  __device__ __forceinline__ void from_acc(const f32x4* acc) {
#pragma unroll
    for (int ct = 0; ct < C / 16; ++ct) v[ct] = acc[ct];
  }
};

// The float32 embedding of one pair formed straight in the channel layout of
// CFrag (lane group g: channels 16 ct + 4 g + r), with write_embedding's
// arithmetic: channel c < C / 2 is the sine of frequency c, channel C / 2 + c
// its cosine. With C a multiple of 32 a lane's channels are the sines and
// cosines of the same C / 8 frequencies.
template <int C>
__device__ __forceinline__ CFrag<float, C> embed_cfrag(float4 pi, float4 pj, const FreqTable& ft, int g) {
  static_assert(C % 32 == 0, "each lane holds the sine and cosine of its frequencies");
  constexpr int FT = C / 32;  // sine channel tiles
  const double x = pair_angle_f64(pi, pj);
  CFrag<float, C> e;
#pragma unroll
  for (int ct = 0; ct < FT; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int f = 16 * ct + 4 * g + r;
      const double rev = x * ((double)ft.ghi[f] + (double)ft.glo[f]);
      const float rr = (float)(rev - __builtin_floor(rev));
      e.v[ct][r] = __builtin_amdgcn_sinf(rr);
      e.v[FT + ct][r] = __builtin_amdgcn_cosf(rr);
    }
  return e;
}

template <int C>
__device__ __forceinline__ f32x4 mma_c(const CFrag<bf16, C>& a, const CFrag<bf16, C>& b, f32x4 c) {
#pragma unroll
  for (int ct = 0; ct < C / 16; ++ct) c = mfma_x16(a.v[ct], b.v[ct], c);
  return c;
}
template <int C>
__device__ __forceinline__ f32x4 mma_c(const CFrag<float, C>& a, const CFrag<float, C>& b, f32x4 c) {
#pragma unroll
  for (int ct = 0; ct < C / 16; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) c = mfma_f32(a.v[ct][r], b.v[ct][r], c);
  return c;
}

// Projection of one row's heads onto the channels, in fp32 MFMA:
//   acc[ct] = (x_row[h] * mult) @ W[:, 16ct..16ct+15]  as U^T[c, h]
// lane (g, n = h) ends with channels 16ct + 4g + r. Step s contracts
// d = (D/4) g + s (lane group g holds a contiguous quarter of the row).
// x_row points at head 0 of the row; hstride = element stride between heads.
template <typename T, int D, int C>
__device__ __forceinline__ void project_row(const T* x_row, long hstride, bool valid, float mult,
                                            const float* __restrict__ W, int g, int n, f32x4* acc) {
  constexpr int Q = D / 4;
  float xv[Q];
  if (valid) {
    const T* p = x_row + n * hstride + Q * g;
#pragma unroll
    for (int s = 0; s < Q; ++s) xv[s] = (float)p[s] * mult;
  } else {
#pragma unroll
    for (int s = 0; s < Q; ++s) xv[s] = 0.f;
  }
#pragma unroll
  for (int ct = 0; ct < C / 16; ++ct) {
    f32x4 a = zero4();
#pragma unroll
    for (int s = 0; s < Q; ++s) a = mfma_f32(W[(Q * g + s) * C + 16 * ct + n], xv[s], a);
    acc[ct] = a;
  }
}

// Pair embedding of one (row i, key j) into an LDS row: channel f is
// sin(x_ij f_f), channel C/2 + f is cos(x_ij f_f) (reference.py:75-84 order).
// bf16 kernels evaluate the angle in fp32 (the result is rounded to bf16);
// fp32 kernels evaluate angle and argument reduction in binary64. With
// SPLIT > 1, SPLIT lanes share the pair: this one writes the frequencies
// [part F / SPLIT, (part + 1) F / SPLIT) and their cosines.
template <typename T, int C, int SPLIT = 1>
__device__ __forceinline__ void write_embedding(T* erow, float4 pi, float4 pj, const FreqTable& ft, int part = 0) {
  constexpr int F = C / 2, FP = F / SPLIT;
  static_assert(FP % 4 == 0, "each lane writes whole groups of four frequencies");
  const int f0 = SPLIT == 1 ? 0 : part * FP;
  float sv[FP], cv[FP];
  if constexpr (is_bf16<T>::value) {
    const float x = pair_angle(pi, pj);
#pragma unroll
    for (int f = 0; f < FP; ++f)
      sincos_rev<false>(x, ft.ghi[f0 + f], ft.glo[f0 + f], (ft.reduce_mask >> (f0 + f)) & 1u, sv[f], cv[f]);
  } else {
    const double x = pair_angle_f64(pi, pj);
#pragma unroll
    for (int f = 0; f < FP; ++f) {
      const double rev = x * ((double)ft.ghi[f0 + f] + (double)ft.glo[f0 + f]);
      const float r = (float)(rev - __builtin_floor(rev));
      sv[f] = __builtin_amdgcn_sinf(r);
      cv[f] = __builtin_amdgcn_cosf(r);
    }
  }
  if constexpr (is_bf16<T>::value) {
#pragma unroll
    for (int f = 0; f < FP; f += 4) {
      bf16x4 a, b;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a[e] = (bf16)sv[f + e];
        b[e] = (bf16)cv[f + e];
      }
      *reinterpret_cast<bf16x4*>(erow + f0 + f) = a;
      *reinterpret_cast<bf16x4*>(erow + F + f0 + f) = b;
    }
  } else {
#pragma unroll
    for (int f = 0; f < FP; f += 4) {
      *reinterpret_cast<f32x4*>(erow + f0 + f) = f32x4{sv[f], sv[f + 1], sv[f + 2], sv[f + 3]};
      *reinterpret_cast<f32x4*>(erow + F + f0 + f) = f32x4{cv[f], cv[f + 1], cv[f + 2], cv[f + 3]};
    }
  }
}

// Lane assignment of a wave's embeddings: NP (row, key) pairs of a chunk
// per wave. NP >= 64: EPL pairs per lane, lane l taking key l % KC of rows
// l / KC + (64 / KC) k; NP < 64 (a divisor of 64): SPLIT = 64 / NP lanes
// per pair, each writing 1 / SPLIT of the frequencies.
template <int NP>
struct EmbedLanes {
  static constexpr bool OK = NP % 64 == 0 || 64 % NP == 0;
  static constexpr int EPL = NP >= 64 ? NP / 64 : 1;
  static constexpr int SPLIT = NP >= 64 ? 1 : 64 / NP;
  // pair slot and frequency part of a lane
  static __device__ __forceinline__ int slot(int lane) { return SPLIT == 1 ? lane : lane % NP; }
  static __device__ __forceinline__ int part(int lane) { return SPLIT == 1 ? 0 : lane / NP; }
};

// Zero the outputs of padding rows [max(row0, len), end) of a padded event,
// where end is the block's last row, or L for the event's last block
// (pad-row contract: forward.py:19-22, 288-304). Rows of out are addressed
// by ra, those of vec_out by rv.
template <typename T>
__device__ __forceinline__ void zero_pad_rows(const EventSpec& ev, const EventBlock& eb, const RowAddr& ra,
                                              const RowAddr& rv, int row0, int rows, int width, int tid,
                                              int nthreads, T* out, float* vec_out, int vec_count) {
  if (ev.packed) return;
  const int nblk = eb.len > 0 ? (eb.len + rows - 1) / rows : 1;
  const int first = row0 > eb.len ? row0 : eb.len;
  const int end = (eb.blk == nblk - 1) ? ev.L : (row0 + rows < ev.L ? row0 + rows : ev.L);
  if (first >= end) return;
  const int nrows = end - first;
  const int total = ev.H * nrows * width;
  for (int idx = tid; idx < total; idx += nthreads) {
    const int c = idx % width;
    const int r = (idx / width) % nrows;
    const int h = idx / (width * nrows);
    out[ra.off(h, first + r, width) + c] = (T)0.f;
  }
  if (vec_out)
    for (int idx = tid; idx < ev.H * nrows * vec_count; idx += nthreads) {
      const int r = (idx / vec_count) % nrows;
      const int h = idx / (vec_count * nrows);
      vec_out[rv.vec(h, first + r) * vec_count + idx % vec_count] = 0.f;
    }
}

// Forward dispatch per (dtype, D), one translation unit each
// (fst_fwd_inst.hip). With query set, only reports the rows per workgroup
// of the kernel that (HP, C) selects (0 = unsupported) in *rows.
// fwd_plans_* reports the FST_PLAN_FWD_* bits compiled for (HP, C).
#define FST_DECL_FWD(NAME)                                                                                       \
  int fwd_dispatch_##NAME(const FwdParams& prm, int HP, int C, hipStream_t stream, int grid, bool query, int* rows); \
  int fwd_plans_##NAME(int HP, int C);
FST_DECL_FWD(bf16_16)
FST_DECL_FWD(bf16_32)
FST_DECL_FWD(bf16_48)
FST_DECL_FWD(bf16_64)
FST_DECL_FWD(f32_16)
FST_DECL_FWD(f32_32)
FST_DECL_FWD(f32_48)
FST_DECL_FWD(f32_64)
#undef FST_DECL_FWD

// Backward dispatch per (dtype, D) (fst_bwd_inst.hip). which = 0: rows
// kernel, 1: cols kernel. With query set, reports rows (or keys) per
// workgroup in *rows (0 = unsupported). bwd_plans_* reports the
// FST_PLAN_ROWS_* / FST_PLAN_COLS_* bits compiled for (HP, C).
#define FST_DECL_BWD(NAME)                                                                                   \
  int bwd_dispatch_##NAME(const BwdParams& prm, int which, int HP, int C, hipStream_t stream, int grid, bool query, \
                          int* rows);                                                                        \
  int bwd_plans_##NAME(int HP, int C);
FST_DECL_BWD(bf16_16)
FST_DECL_BWD(bf16_32)
FST_DECL_BWD(bf16_48)
FST_DECL_BWD(bf16_64)
FST_DECL_BWD(f32_16)
FST_DECL_BWD(f32_32)
FST_DECL_BWD(f32_48)
FST_DECL_BWD(f32_64)
#undef FST_DECL_BWD

// ---------------------------------------------------------------------------
// Plan requests of the first-generation kernels (fst_forward.hip,
// fst_backward.hip), which come in (NW, NS) splits: NW waves per 16-row tile
// (16 * 4 / NW rows or keys per four-wave workgroup; NW = 8 is one 16-row
// tile in an eight-wave workgroup) and 16 * NS keys (or rows) per chunk.
// ---------------------------------------------------------------------------
// (NW, NS) of a plan request for a family of configurations F<NW, NS>
// (nw, ns = 0: not requested), as 10 NW + NS, or 0 when nothing fits.
// Preference: the most waves per 16-row tile first (on gfx950 the 16-row
// workgroups run about twice as fast as 64-row ones, e.g. 2.8 against 5.3
// ms for the float32 forward at B=256, L=768, H=12, D=32, C=16: more waves
// share the tile's work and each holds less), then ns_first keys (or rows)
// per chunk.
template <template <int, int> class F>
constexpr int pick_split(int nw, int ns, int ns_first = 2) {
  const bool fits[4][2] = {{F<8, 1>::FITS, F<8, 2>::FITS}, {F<4, 1>::FITS, F<4, 2>::FITS},
                           {F<2, 1>::FITS, F<2, 2>::FITS}, {F<1, 1>::FITS, F<1, 2>::FITS}};
  const int nws[4] = {8, 4, 2, 1};
  for (int w = 0; w < 4; ++w) {
    if (nw && nws[w] != nw) continue;
    for (int k = 0; k < 2; ++k) {
      const int s = k == 0 ? ns_first : 3 - ns_first;
      if (ns && s != ns) continue;
      if (fits[w][s - 1]) return 10 * nws[w] + s;
    }
  }
  return 0;
}

// The requested (nw, ns) of the plan bits in flags, for the groups starting
// at bit t (three tile-height bits) and bit k (two key-chunk bits).
// t: bit index of the T16 / T32 / T64 triple; w8: bit index of the
// eight-wave 16-row tile.
__host__ __device__ inline int plan_nw(int flags, int t, int w8) {
  return (flags >> w8) & 1 ? 8
                           : ((flags >> t) & 1 ? 4 : ((flags >> (t + 1)) & 1 ? 2 : ((flags >> (t + 2)) & 1 ? 1 : 0)));
}
__host__ __device__ inline int plan_ns(int flags, int k) { return (flags >> k) & 1 ? 1 : ((flags >> (k + 1)) & 1 ? 2 : 0); }
constexpr int bit_index(int b) { return b <= 1 ? 0 : 1 + bit_index(b >> 1); }

// The plan bits of a (NW, NS) family: a tile-height bit for each NW and a
// key-chunk bit for each NS that fits with some value of the other.
template <template <int, int> class F>
constexpr int split_plans(int t16, int k16, int w8) {
  int bits = 0;
  const int nws[3] = {4, 2, 1};
  for (int w = 0; w < 3; ++w)
    if (pick_split<F>(nws[w], 0)) bits |= t16 << w;
  if (pick_split<F>(8, 0)) bits |= w8;
  for (int s = 1; s <= 2; ++s)
    if (pick_split<F>(0, s)) bits |= k16 << (s - 1);
  return bits;
}

}  // namespace fst
