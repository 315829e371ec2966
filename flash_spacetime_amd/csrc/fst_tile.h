// Building blocks of the second-generation gfx950 kernels (one 16-row tile
// per workgroup, four waves, operands straight from global memory).
//
// Layout conventions are those of fst_device.h (lane = 16 g + n, MFMA A / B /
// C layouts). On top of them:
//  * Channel slots. The C embedding channels of a pair are contracted in
//    16-slot steps ct (16x16x16 bf16). Slot k = 16 ct + 4 g + e of lane group
//    g holds, for e = 0, 1, sin(x f) and for e = 2, 3, cos(x f) of frequency
//    f = 8 ct + 2 g + (e & 1), so every lane evaluates two sin/cos pairs per
//    step from one angle. `slot_channel` maps a slot to the spec's channel
//    index (sin channels first, then cos: reference.py:82-84); the weight is
//    read through it wherever a slot meets W, so the permutation never shows
//    outside the kernels.
//  * Transposes on the matrix core. An operand tile held as A (lane n = row,
//    slots = four columns of group g) multiplied by the identity gives the
//    tile in C layout with the roles swapped (lane n = column, registers =
//    rows 4g .. 4g+3), which is again an A / B operand of a 16x16x16 step
//    after packing to bf16. The values are bf16 inputs times 1 plus zeros,
//    so the transpose is exact.
//  * LDS layouts are swizzled so that every access pattern below touches 64
//    distinct banks per pass (gfx950: 64 banks of 4 bytes).
#pragma once

#include <type_traits>

#include "fst_kernels.h"

namespace fst {

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Hardware workgroup w of a grid of G (a multiple of 8) runs logical block
// (w % 8) * (G / 8) + w / 8: workgroups are dealt to the eight XCDs round
// robin, so each XCD gets a contiguous range of logical blocks and an event's
// row blocks share one L2.
__device__ __forceinline__ int xcd_remap(int w, int G) { return (w & 7) * (G >> 3) + (w >> 3); }

// Natural channel index of channel slot k (see the header comment).
template <int C>
__host__ __device__ constexpr int slot_channel(int k) {
  const int ct = k >> 4, g = (k >> 2) & 3, e = k & 3;
  const int f = 8 * ct + 2 * g + (e & 1);
  return e < 2 ? f : C / 2 + f;
}

// Frequencies whose largest angle 4096 f / (2 pi) leaves the +-256 revolution
// domain of v_sin_f32 / v_cos_f32: f_k > 0.3927, i.e. the first C / 16 of the
// ladder exp(-k ln(1e4) / (C/2)). They sit in channel step 0.
template <int C>
struct EmbedSteps {
  static constexpr int NCT = C / 16;
  static constexpr int NRED = C / 16;
  // In step 0, lane group 0 holds frequencies 0 and 1, group 1 holds 2 and 3.
  static constexpr bool RA = NRED >= 1;  // frequency 2g needs reduction for some g
  static constexpr bool RB = NRED >= 2;  // frequency 2g + 1 needs reduction for some g
};


// clip(sign(I) sqrt|I|, -4, 4) for I = |p_i - p_j|^2 - (18 (t_i - t_j))^2:
// the spec's pair angle (reference.py:75-81) without its factor 1024, which
// the frequencies carry (a power of two, so no rounding moves).
__device__ __forceinline__ float pair_angle_unit(float4 a, float4 b) {
  const float dx = a.x - b.x, dy = a.y - b.y, dz = a.z - b.z;
  const float dt = (a.w - b.w) * kTimeScale;
  const float interval = __builtin_fmaf(dx, dx, __builtin_fmaf(dy, dy, __builtin_fmaf(dz, dz, -dt * dt)));
  const float mag = __builtin_amdgcn_sqrtf(fabsf(interval));
  return __builtin_amdgcn_fmed3f(__builtin_copysignf(mag, interval), -kClip, kClip);
}

// x of every lane group, gathered into every lane: out[r] = x of lane group r
// (same n). v_permlane32_swap exchanges lanes 32-63 of its first operand with
// lanes 0-31 of its second, v_permlane16_swap the odd 16-lane rows of the
// first with the even rows of the second.
__device__ __forceinline__ void group_gather(float x, float out[4]) {
  const unsigned u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);  // x_{g&1}, x_{2+(g&1)}
  const auto b = __builtin_amdgcn_permlane16_swap(a[0], a[0], false, false);
  const auto c = __builtin_amdgcn_permlane16_swap(a[1], a[1], false, false);
  out[0] = __uint_as_float(b[0]);
  out[1] = __uint_as_float(b[1]);
  out[2] = __uint_as_float(c[0]);
  out[3] = __uint_as_float(c[1]);
}


// The four embedding slots of lane group g in channel step ct for one pair
// angle x (unit angle): {sin x fa, sin x fb, cos x fa, cos x fb}, fa and fb
// the lane's frequencies times 1024 / (2 pi) (revolutions per unit angle).
// RA / RB reduce the argument to [0, 1) revolutions first (the channels of
// step 0 whose frequency can leave the +-256 revolution domain).
template <bool RA, bool RB>
__device__ __forceinline__ bf16x4 embed_slots(float x, float fa, float fb) {
  float pa = x * fa, pb = x * fb;
  if constexpr (RA) pa = __builtin_amdgcn_fractf(pa);
  if constexpr (RB) pb = __builtin_amdgcn_fractf(pb);
  const f32x4 e{__builtin_amdgcn_sinf(pa), __builtin_amdgcn_sinf(pb), __builtin_amdgcn_cosf(pa),
                 __builtin_amdgcn_cosf(pb)};
  return pack4(e);
}

template <int C>
__device__ __forceinline__ bf16x4 embed_step(float x, float fa, float fb, int ct) {
  if (ct == 0) return embed_slots<EmbedSteps<C>::RA, EmbedSteps<C>::RB>(x, fa, fb);
  return embed_slots<false, false>(x, fa, fb);
}

// Identity operand of a 16x16x16 step: lane (g, n) slot e = [4 g + e == n].
__device__ __forceinline__ bf16x4 ident_x16(int g, int n) {
  bf16x4 id;
#pragma unroll
  for (int e = 0; e < 4; ++e) id[e] = (bf16)((4 * g + e == n) ? 1.f : 0.f);
  return id;
}


// Transpose of a 16x16 tile held as an A operand (lane n = row m, slots =
// columns 4g .. 4g+3): lane n now holds column n, slots = rows 4g .. 4g+3.
__device__ __forceinline__ bf16x4 transpose_x16(bf16x4 a, bf16x4 id) { return pack4(mfma_x16(a, id, zero4())); }

// Lower / upper four slots of a 16x16x32 operand.
__device__ __forceinline__ bf16x4 lo4(const bf16x8& v) { return __builtin_shufflevector(v, v, 0, 1, 2, 3); }
__device__ __forceinline__ bf16x4 hi4(const bf16x8& v) { return __builtin_shufflevector(v, v, 4, 5, 6, 7); }
__device__ __forceinline__ bf16x8 cat8(const bf16x4& a, const bf16x4& b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Head-dim tiles of an operand loaded as KFrag<bf16, D> (lane n = row, group
// g holds the feature slots of fst_device.h) after transposing: tile q holds
// feature dmap(q, g', r) in register r of lane group g' of the product it is
// contracted into. 16x16x32 fragments (D % 32 == 0) split each 32-feature
// step t into its lower and upper four slots (tiles 2t, 2t+1); 16x16x16
// fragments map one to one.
template <int D>
struct DTiles {
  static constexpr bool X32 = (D % 32) == 0;
  static constexpr int NQ = D / 16;
  static __device__ __forceinline__ int dmap(int q, int g, int r) {
    if constexpr (X32) return 32 * (q >> 1) + 8 * g + 4 * (q & 1) + r;
    else return 16 * q + 4 * g + r;
  }
  // A-operand half tile q of a fragment (16 rows x 16 features).
  static __device__ __forceinline__ bf16x4 part(const KFrag<bf16, D>& f, int q) {
    if constexpr (X32) return (q & 1) ? hi4(f.x32[q >> 1]) : lo4(f.x32[q >> 1]);
    else return f.x16[q];
  }
};

// ---------------------------------------------------------------------------
// Work items of the 16-row tile kernels. Padded events map directly: logical
// block w is tile w % nb of event w / nb (nb = ceil(L / 16)), so a tile wholly
// past its event's length only zeroes its rows. Packed events have no padding
// and use prefix sums of their tile counts.
// ---------------------------------------------------------------------------
//
// Packed schedule. The events' tiles are listed longest event first (ev.perm,
// prefix sums ev.scum) and dealt to the XCDs in groups of eight consecutive
// tiles, round robin: XCD x takes groups x, x + 8, x + 16, ... A tile's cost
// grows with its event's length, so neighbouring groups cost about the same
// and every XCD gets an equal share of each length class, longest first,
// while the eight tiles of a group share their event's K and V in one L2.
// Hardware workgroup w runs on XCD w % 8 as its (w / 8)-th tile; the grid is
// a multiple of 64.
//
// Padded schedule. Every padded event has nb tiles, so the work of an event
// grows with its length squared while its tile count does not: events are
// taken by decreasing length (ev.perm) and dealt to the eight XCDs in snake
// order (ranks 8j .. 8j+7 go to XCDs 0..7 for even j, 7..0 for odd j), which
// balances the XCDs' work and starts the longest events first. Workgroups
// are dealt to the XCDs round robin, so hardware workgroup w runs on XCD
// w % 8 as its (w / 8)-th tile: tile (w / 8) % nb of the XCD's (w / 8) / nb-th
// event. The grid is 8 ceil(B / 8) nb. With ev.vp (the rows kernel) each
// XCD runs its events' valid tiles first and their padding-only tiles, which
// only write zeros, after them: at two workgroups per CU those held one of
// the CU's two slots between the events (cfg2 rows kernel 0.736 -> 0.713 ms;
// the forward and cols kernel, at three per CU, keep the interleaved order,
// which measured 1 % faster for them).
__device__ __forceinline__ bool tile_block(const EventSpec& ev, int w, EventBlock& eb) {
  if (ev.packed) {
    if (!ev.scum) return locate_block(ev, xcd_remap(w, gridDim.x), eb);
    const int x = w & 7, k = w >> 3;
    const int t = (((k >> 3) << 3) + x) * 8 + (k & 7);
    if (t >= ev.scum[ev.B]) return false;
    const int32_t* sc = ev.scum;
    const int lo = wave_last_le(ev.B, t, [&](int i) { return sc[i]; });
    eb.b = ev.perm[lo];
    eb.blk = t - ev.scum[lo];
    event_range(ev, eb.b, eb.tok0, eb.len);
    return true;
  }
  const int nb = (ev.L + 15) >> 4;
  const int x = w & 7, k = w >> 3;
  int j, blk;
  if (ev.vp) {
    // Padding-last: XCD x takes the valid tiles of its events (same events,
    // same order) first and their padding-only tiles after them. v[j] - v[0]
    // counts the valid tiles of the XCD's first j events, so those events'
    // padding tiles number j nb - (v[j] - v[0]) (every real event has nb
    // tiles). Workgroups past both lists have no tile.
    const int S = (ev.B + 7) >> 3;
    const int32_t* v = ev.vp + x * S;
    const int base = v[0], tv = v[S] - base;
    if (k < tv) {
      j = wave_last_le(S, k + base, [&](int i) { return v[i]; });  // v[j] - base <= k < v[j + 1] - base
      blk = k - (v[j] - base);
    } else {
      const int q = k - tv, jb = ev.B >> 3;
      // XCD x's real events: the full groups of eight ranks, and the last
      // partial group's rank when it exists.
      const int jr = jb + ((((jb & 1) ? 7 - x : x) < (ev.B & 7)) ? 1 : 0);
      if (q >= jr * nb - tv) return false;
      // padding tiles of the events before j <= q < those of the events up to j
      j = wave_last_le(jr, q - base, [&](int i) { return i * nb - v[i]; });
      blk = (v[j + 1] - v[j]) + (q - (j * nb - (v[j] - base)));
    }
  } else {
    j = k / nb;
    blk = k - j * nb;
  }
  const int r = 8 * j + ((j & 1) ? 7 - x : x);
  if (r >= ev.B) return false;
  const int b = ev.perm[r];
  eb.b = b;
  eb.blk = blk;
  event_range(ev, b, eb.tok0, eb.len);
  return true;
}

// Zero rows [max(i0, len), min(i0 + 16, L)) of a padded event for every head
// (pad-row contract: forward.py:19-22), 16 bytes per store, addressed by ra;
// `vec` gets zeros at the same (head, row) positions, addressed by rv, when
// not null.
template <typename T, int D, int NT = 256>
__device__ __forceinline__ void zero_tile_rows(const EventSpec& ev, const RowAddr& ra, const RowAddr& rv, int i0,
                                               int len, int H, int tid, T* out, float* vec) {
  if (ev.packed) return;
  const int first = i0 > len ? i0 : len;
  const int end = i0 + 16 < ev.L ? i0 + 16 : ev.L;
  if (first >= end) return;
  const int nr = end - first;
  constexpr int CH = D * (int)sizeof(T) / 16;
  for (int idx = tid; idx < H * nr * CH; idx += NT) {
    const int c = idx % CH, r = (idx / CH) % nr, h = idx / (CH * nr);
    *reinterpret_cast<u32x4*>(out + ra.off(h, first + r, D) + c * (16 / (int)sizeof(T))) = u32x4{0u, 0u, 0u, 0u};
  }
  if (vec)
    for (int idx = tid; idx < H * nr; idx += NT) vec[rv.vec(idx / nr, first + idx % nr)] = 0.f;
}

// The W operand of project_loaded, split into bf16 parts hi = bf16(W) and
// lo = bf16(W - hi) (W to 16 significant bits): lane (g, n) holds W[Qd g +
// i][channel(16 ct + n)] for its Qd = D / 4 features i, in steps of 8 (16x16x32
// products) where Qd is a multiple of 8, else of 4 (16x16x16). Loaded once
// and shared by every row a kernel projects.
template <int D, int C>
struct WSlots {
  static constexpr int Qd = D / 4, STEP = Qd % 8 == 0 ? 8 : 4, NST = Qd / STEP;
  using V = std::conditional_t<STEP == 8, bf16x8, bf16x4>;
  V hi[C / 16][NST], lo[C / 16][NST];
  __device__ __forceinline__ void load(const float* __restrict__ W, int g, int n) {
#pragma unroll
    for (int ct = 0; ct < C / 16; ++ct)
#pragma unroll
      for (int st = 0; st < NST; ++st)
#pragma unroll
        for (int e = 0; e < STEP; ++e) {
          const float wv = W[(Qd * g + STEP * st + e) * C + slot_channel<C>(16 * ct + n)];
          const bf16 h = (bf16)wv;
          hi[ct][st][e] = h;
          lo[ct][st][e] = (bf16)(wv - (float)h);
        }
  }
};

// One row's operand of a projection: features Qd g .. Qd g + Qd - 1 of head
// n's row in 8- or 16-byte loads (a row holds D bf16, so they are aligned); a
// lane with !ok reads head 0. Loading is apart from projecting so a kernel
// can issue the loads of all its rows before the first product waits on one.
template <int D>
struct SlotRow {
  static constexpr int Qd = D / 4, VW = Qd % 8 == 0 ? 8 : 4, NV = Qd / VW;
  using V = std::conditional_t<VW == 8, bf16x8, bf16x4>;
  V x[NV];
  __device__ __forceinline__ void load(const bf16* xrow, long hstride, bool ok, int g, int n) {
    const bf16* p = xrow + (ok ? n * hstride : 0) + Qd * g;
#pragma unroll
    for (int t = 0; t < NV; ++t) x[t] = *reinterpret_cast<const V*>(p + VW * t);
  }
};

// u = bf16(mult (x @ W[:, channel(slot)])) for the heads of one row (x =
// q with mult = scale, or dO with mult = 1): bf16 MFMA over x (exact in bf16)
// and W's two parts, accumulated in fp32, so the product keeps W to 16 bits
// before the one rounding to bf16; the head is on lane n (heads >= H or an
// invalid row give zeros) and lane (g, n = h) receives slots 16 ct + 4 g .. +3.
template <int D, int C>
__device__ __forceinline__ void project_loaded(const SlotRow<D>& xr, bool ok, float mult, const WSlots<D, C>& wv,
                                            bf16x4* out) {
  using WS = WSlots<D, C>;
  static_assert(SlotRow<D>::VW == WS::STEP, "one SlotRow vector per product step");
#pragma unroll
  for (int ct = 0; ct < C / 16; ++ct) {
    f32x4 a = zero4();
#pragma unroll
    for (int st = 0; st < WS::NST; ++st) {
      const typename WS::V x = ok ? xr.x[st] : typename WS::V{};
      if constexpr (WS::STEP == 8) {
        a = mfma_x32(wv.hi[ct][st], x, a);
        a = mfma_x32(wv.lo[ct][st], x, a);
      } else {
        a = mfma_x16(wv.hi[ct][st], x, a);
        a = mfma_x16(wv.lo[ct][st], x, a);
      }
    }
    out[ct] = pack4(a * mult);
  }
}

// fp32 quad -> bf16 parts hi = bf16(x), lo = bf16(x - hi) (x to 16 bits).
__device__ __forceinline__ void split4(const f32x4& x, bf16x4& hi, bf16x4& lo) {
  hi = pack4(x);
  f32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = x[e] - (float)hi[e];
  lo = pack4(r);
}

// C += A B over 16 k-slots (16x16x16 operand layouts) with A and B given as
// bf16 parts: three products, lo x lo (below 2^-16 of the result) dropped.
__device__ __forceinline__ f32x4 mma_split(bf16x4 ah, bf16x4 al, bf16x4 bh, bf16x4 bl, f32x4 c) {
  c = mfma_x16(al, bh, c);
  c = mfma_x16(ah, bl, c);
  return mfma_x16(ah, bh, c);
}

// Load and project one row; xrow points at head 0 of the row, hstride is the
// element stride of heads.
template <int D, int C>
__device__ __forceinline__ void project_slots(const bf16* xrow, long hstride, bool ok, float mult,
                                              const WSlots<D, C>& wv, int g, int n, bf16x4* out) {
  SlotRow<D> xr;
  xr.load(xrow, hstride, ok, g, n);
  project_loaded<D, C>(xr, ok, mult, wv, out);
}

// ---------------------------------------------------------------------------
// Layout of the u / w~ scratch the rows kernel writes for the cols kernel.
// Rows are grouped by four ("row group" = a quarter of a 16-row tile; the
// groups of an event start at 4 x its first tile in the rows work list).
// Within a group, for each half (rows 0-1 / 2-3), channel step ct, head h and
// lane group g, the 8 values (row 2 half + rb, slot 16 ct + 4 g + e) sit
// together, rb = 0..1, e = 0..3. A cols-kernel lane (g, head n) then reads two
// rows of its four slots with one 16-byte load, and the 64 lanes of the load
// read one contiguous run; a row-major [rows, H, C] layout would put the
// heads of one row an entire head plane apart.
// ---------------------------------------------------------------------------
__device__ __forceinline__ long uw_group_elems(int H, int NCT) { return 64L * NCT * H; }
__device__ __forceinline__ int uw_off(int half, int ct, int h, int g, int rb, int H, int NCT) {
  return (((half * NCT + ct) * H + h) * 4 + g) * 8 + rb * 4;
}

// ---------------------------------------------------------------------------
// Buffer loads. One resource per tensor and event (base = the event's first
// element, range = its bytes); a lane's offset within the event is fixed and
// the key chunk moves through the scalar offset, so the chunk loop spends no
// vector instructions on addresses. Offsets past the range read as zero.
// ---------------------------------------------------------------------------
struct Buf {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ Buf(const void* base, unsigned bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000)) {}
  __device__ __forceinline__ bf16x8 ld128(int voff, int soff) const {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  }
  __device__ __forceinline__ bf16x4 ld64(int voff, int soff) const {
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
  }
  __device__ __forceinline__ float4 ldf4(int voff, int soff) const {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  }
  __device__ __forceinline__ float ldf(int voff, int soff) const {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
  }
};

// Byte offset of lane group g's part of a KFrag<bf16, D> row, and the loader:
// 16x16x32 steps t at 64 t + 16 g, 16x16x16 steps at 32 t + 8 g.
template <int D>
__device__ __forceinline__ int kfrag_goff(int g) {
  return (D % 32 == 0) ? 16 * g : 8 * g;
}
template <int D>
__device__ __forceinline__ void load_kfrag(KFrag<bf16, D>& f, const Buf& b, int voff, int soff) {
#pragma unroll
  for (int t = 0; t < KFrag<bf16, D>::N32; ++t) f.x32[t] = b.ld128(voff + 64 * t, soff);
#pragma unroll
  for (int t = 0; t < KFrag<bf16, D>::N16; ++t) f.x16[t] = b.ld64(voff + 32 * t, soff);
}

// K / V (or streamed) rows staged through LDS by the wave that uses them:
// buffer loads write LDS directly, so nothing occupies VGPRs while the next
// chunk is in flight. A KFrag<bf16, D> of 16 rows (D % 32 == 0) takes D / 32
// blocks of 1 KB; lane l's 16 bytes of block t sit at 16 l. The LDS base of
// a load must be wave-uniform.
template <int D>
struct LdsFrag {
  static_assert(D % 32 == 0, "LDS-staged fragments need 16-byte lane parts");
  static constexpr int NP = D / 32;
  static constexpr int BYTES = NP * 1024;
  static __device__ __forceinline__ void load(const Buf& b, unsigned char* dst, int voff, int soff) {
#pragma unroll
    for (int t = 0; t < NP; ++t)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(b.r, (__attribute__((address_space(3))) void*)(dst + t * 1024), 16,
                                               voff + 64 * t, soff, 0, 0);
  }
  static __device__ __forceinline__ void read(KFrag<bf16, D>& f, const unsigned char* src, int lane) {
#pragma unroll
    for (int t = 0; t < NP; ++t) f.x32[t] = *reinterpret_cast<const bf16x8*>(src + t * 1024 + 16 * lane);
  }
};

// Workgroup barrier for exchanges through LDS: this wave's LDS accesses are
// complete before it. Unlike __syncthreads() it does not wait for the wave's
// outstanding buffer loads, loads into LDS included (the compiler's
// workgroup release fence waits for all of those when any load into LDS is
// in flight); a wave reads what its own loads put in LDS only after waiting
// for them itself.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---------------------------------------------------------------------------
// LDS layouts.
// ---------------------------------------------------------------------------

// Embedding tile: [row 16][ct][key KC][16 slots] bf16. The four 8-byte blocks
// (slot groups) of key j are stored in the order b ^ ((j >> 2) & 3): an
// 8-byte write pass (16 keys of one block, 32 bytes apart) then covers the 32
// banks of a pass once, and a transposing read of 8 keys x 4 blocks covers
// 256 contiguous bytes.
template <int C, int KC>
struct ETile {
  static constexpr int NCT = C / 16;
  static constexpr int BYTES = 16 * NCT * KC * 16 * 2;
  static __device__ __forceinline__ int off(int row, int ct, int key, int blk) {
    return (((row * NCT + ct) * KC + key) << 4) + ((blk ^ ((key >> 2) & 3)) << 2);
  }
  static __device__ __forceinline__ void store(bf16* e, int row, int ct, int key, int g, bf16x4 v) {
    *reinterpret_cast<bf16x4*>(e + off(row, ct, key, g)) = v;
  }
  // Four consecutive keys kb + 4g .. kb + 4g + 3 of channel slot 16 ct + n,
  // through the transposing read (source lane s of the group supplies key
  // kb + 4g + s / 4, block s % 4).
  static __device__ __forceinline__ bf16x4 load_tr(const bf16* e, int row, int ct, int kb, int g, int n) {
    const bf16* p = e + off(row, ct, kb + 4 * g + (n >> 2), n & 3);
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
  }
};

// Exchange slots between the row-major and head-major roles: 16-byte chunk c
// of slot (row i, head h) at ((c * 16 + i) * 16 + (h ^ i)) * 16 bytes. With
// the head index on the lanes (fixed row) or the row index on the lanes
// (fixed head) the lanes of one LDS pass (8 per 16-byte write, 16 per
// 16-byte read) hit distinct banks. Heads are padded to 16 slots.
__device__ __forceinline__ int stage_off(int c, int i, int h) { return (((c << 4) + i) << 8) + ((h ^ i) << 4); }

// One 8-byte half of such a slot (P and dS, bf16): half `half` of lane group
// g & 1, swapped when (h ^ i) >= 8, so that the 16 lanes of one 8-byte write
// pass (rows on the lanes) cover the 32 banks of a pass exactly once.
__device__ __forceinline__ int half_off(int c, int i, int h, int half) {
  return stage_off(c, i, h) + ((half ^ (((h ^ i) >> 3) & 1)) << 3);
}

// Operand rows of one 16-row chunk in LDS (qt and dO in the cols kernel): per
// (tensor, head, 32-feature part) a 1 KB block of 16 rows x 4 16-byte
// quarters, quarter c of row r at slot 4 r + (c ^ swz(r)), swz(r) = (r >> 2)
// with its two bits swapped (0, 2, 1, 3). One direct-to-LDS load (lane l ->
// slot l) fills a block. Bank model of gfx950 LDS reads (256 bytes a pass:
// 16 lanes of a 16-byte read, 32 of an 8-byte read): the 16-byte read of
// quarter g by a lane group's 16 rows covers the pass once because swz is a
// permutation of r >> 2; the transposing 8-byte read of 16-feature slice q
// takes quarters 2q, 2q + 1 of rows 0-7 (or 8-15) in one pass, and rows r,
// r + 4 (which share banks) find them at quarters 2q ^ 2, 2q ^ 3 of each
// other, since swz(r) ^ swz(r + 4) = 2 for those rows.
struct QoTile {
  static __device__ __forceinline__ int swz(int r) { return ((r >> 1) & 2) | ((r >> 3) & 1); }
  static __device__ __forceinline__ int slot(int r, int c) { return 4 * r + (c ^ swz(r)); }
  // Row-major fragment part (row n, features 8g .. 8g + 7 of the part).
  static __device__ __forceinline__ bf16x8 row_frag(const unsigned char* blk, int g, int n) {
    return *reinterpret_cast<const bf16x8*>(blk + 16 * slot(n, g));
  }
  // Transposed 16x16 operand of 16-feature slice q & 1 of the part (features
  // 16 (q & 1) .. +15, quarters 2 (q & 1) and 2 (q & 1) + 1): lane (g, n)
  // receives rows 4g .. 4g + 3 of feature 16 (q & 1) + n of the part. Source
  // lane s of the group supplies row 4g + s / 4, features 16 (q & 1) +
  // 4 (s % 4) .. +3.
  static __device__ __forceinline__ bf16x4 tr_frag(const unsigned char* blk, int q, int g, int n) {
    const int r = 4 * g + (n >> 2), j = n & 3;
    const unsigned char* p = blk + 16 * slot(r, 2 * (q & 1) + (j >> 1)) + 8 * (j & 1);
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
  }
  // The same operand with the features in the order of DTiles::dmap: lane
  // (g, n) receives rows 4g .. 4g + 3 of feature 8 (n >> 2) + 4 (q & 1) +
  // (n & 3) of the part. Source lane s of the group supplies row 4g + s / 4,
  // features 8 (s % 4) + 4 (q & 1) .. +3 (half q & 1 of quarter s % 4).
  static __device__ __forceinline__ bf16x4 tr_frag_dmap(const unsigned char* blk, int q, int g, int n) {
    const unsigned char* p = blk + 16 * slot(4 * g + (n >> 2), n & 3) + 8 * (q & 1);
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
  }
};

// Per-(row, head) scalars (rescale factors): [head][17].
__device__ __forceinline__ int scal_off(int i, int h) { return (h * 17 + i) << 2; }

}  // namespace fst
