// Backward kernels of flash-spacetime attention for gfx950, bf16 operands.
//
// Gradients of the spec (reference.py:106-167) in the fused form of
// backward.py:3-32. With qt = bf16(q*scale), u = bf16(qt W), w~ = bf16(dO W),
// dob = dO.b:
//   s_ij  = qt_i.k_j + [A] u_i.E_ij,          P_ij = exp(s_ij - lse_i)
//   dP_ij = dO_i.v_j + [V] (w~_i.E_ij + dob_i)
//   D_i   = sum_j P_ij dP_ij / sum_j P_ij     (from the same P and dP as dS)
//   dS_ij = P_ij (dP_ij - D_i)
//   dq_i  = scale (sum_j dS_ij k_j + [A] (W H_i + sigma_i b))
//   dk_j  = sum_i dS_ij qt_i,      dv_j = sum_i P_ij dO_i
//   dW    = [A] sum qt (x) H + [V] sum dO (x) G,  H_i = sum_j dS_ij E_ij,
//           G_i = sum_j P_ij E_ij,  sigma_i = sum_j dS_ij,  db = [V] sum dO
//
// Rows kernel (one 16-row tile per workgroup, roles as in the forward): a
// single pass over the keys. D is formed online: after chunk t the running
// D_t = N_t / Z_t (N = sum P dP, Z = sum P over the keys seen) replaces
// D_{t-1}, and the accumulators built with the old value are corrected with
// the sums of P they lack, dQ -= (D_t - D_{t-1}) sum P k and H -= (D_t -
// D_{t-1}) G, before chunk t adds P (dP - D_t) terms. At the end every
// accumulator equals its value for D = N / Z over all keys, the same N and Z
// that give sigma = N - D Z; a fully peaked row (all mass on one key) has
// D_t = dP of that key from its chunk on, so its dS vanishes as in the
// two-pass form (backward.py:371-407). Given the forward's output, dS is
// formed against a fixed reference instead, D_ref = dO . (out - [V] b) (D up
// to the output's rounding), each lane keeps its part of N and Z, and the
// correction is made once after the last chunk with D = N / Z: dQ -= (D -
// D_ref) sum P k, H -= (D - D_ref) G. Either way D is the kernel's own N / Z.
// Every accumulator is then divided by Z (P / Z instead of P: the forward's
// rounded lse leaves a common factor on a row's P, which Z measures), and
// the cols kernel recomputes the same normalised P from lse_z = lse log2 e
// + log2 Z.
// The row constant dob never enters a
// pair: with dP~ = dP - dob, D - dob = sum P dP~ / sum P and dS = P (dP~ -
// (D - dob)), so the kernel forms D - dob directly. It writes qt, u, w~ and
// D - dob for the cols kernel and a per-tile dW / db partial.
//
// Cols kernel (one 16-key tile per workgroup, rows streamed): S = Qt K^T and
// dP = dO V^T with the keys on the lanes, dV^T += dO^T P and dK^T += Qt^T dS
// (Qt^T, dO^T read transposed from the chunk's qt / dO rows, which go
// straight to LDS, or made on the matrix core where those do not fit). The
// row-owner part forms
// u_i E_i^T and w~_i E_i^T for the streamed rows with the heads on the
// registers; four consecutive rows of a lane are regrouped in registers so
// that the exchange to the head-owners is one 16-byte write and read per
// (row group, head, key).
//
// The rows kernel runs four waves per workgroup, or eight where a four-wave
// lane's state would spill (Rows2Cfg, Bwd2Pick). Rows are addressed through
// two RowAddr: q, k, v, dq, dk, dv through row_addr_x (their token stride is
// three times the others' when they are the slots of one fused projection),
// dO, the per-row vectors and the scratch through row_addr.
//
// Both kernels write every output exactly once in a fixed order (no atomics),
// so results are bitwise reproducible.
#include "fst_tile.h"

#ifndef FST_ROWS_HB
#define FST_ROWS_HB 1
#endif
#ifndef FST_ROWS_KC
#define FST_ROWS_KC 16
#endif

namespace fst {

// ---------------------------------------------------------------------------
// Rows kernel.
// ---------------------------------------------------------------------------
// NW waves of 64 lanes: 4 (two workgroups per CU), or 8 (one workgroup per
// CU) where the state of a four-wave lane would not fit the registers
// (Bwd2Pick). WPE: waves per SIMD the register plan is built for (2, or 4
// for eight waves in two workgroups per CU). A wave is row-owner of RPW =
// 16 / NW rows and head-owner of HW = ceil(HP / NW) heads, or HW - 1 for
// the waves from NBIG on where NW does not divide HP; waves w and w + 4
// share a SIMD, so with NBIG = 4 every SIMD owns the same number of heads.
template <int HP, int D, int C, int KC, int NW = 4, int WPE = 2, bool KLV = false>
struct Rows2Cfg {
  static constexpr int HW = (HP + NW - 1) / NW, NS = KC / 16, NCT = C / 16, RPW = 16 / NW;
  static constexpr int NBIG = HP - NW * (HW - 1);
  static constexpr int WG_PER_CU = 4 * WPE / NW;
  static constexpr int E_BYTES = ETile<C, KC>::BYTES;
  static constexpr int REGION = (KC / 4) * 16 * 16 * 16;  // one fp32 term of KC keys per (row, 16 head slots)
  // Two per-(row, head slot) scalars: the increments of D (scal_off), and
  // after the key loop the row's 1 / Z (the same offsets in the second half).
  static constexpr int SCAL_BYTES = 2 * 16 * 17 * 4;
  static constexpr int MAIN = E_BYTES + 2 * REGION + SCAL_BYTES;
  // Epilogue: the tile's qt and dO rows, then four dW / db partials (one per
  // wave, or per pair of waves w, w + 4) in the same bytes; one channel step
  // of H (or G) after them, each wave's rows its own.
  static constexpr int DW_BYTES = 4 * (D * C + D) * 4;
  // The rows are staged [op][head][16 rows of XS_RS + pad] (bf16): the dW
  // products read four rows of one head and feature per lane with one
  // transposing read, and these strides put lane groups 0 and 1 (2 and 3),
  // which share an LDS phase, on disjoint banks.
  static constexpr int XS_RS = D == 64 ? 80 : D;                     // row stride
  static constexpr int XS_HS = 16 * XS_RS + (D == 32 ? 16 : 64);     // head stride
  static constexpr int XS_BYTES = HP * XS_HS * 2;
  static constexpr int X_DW = DW_BYTES > 2 * XS_BYTES ? DW_BYTES : 2 * XS_BYTES;
  static constexpr int HG_BYTES = 16 * HP * 16 * 4;
  static constexpr int EPI = X_DW + HG_BYTES;
  static constexpr int LDS_BYTES = MAIN > EPI ? MAIN : EPI;  // dynamic
  // KL (FST_PLAN_ROWS_KV_LDS): each chunk's K and V rows go straight to LDS
  // (QoTile blocks, one per tensor, head and 32-feature part), where D is a
  // multiple of 32, the chunk 16 keys and the blocks fit the LDS share. S and
  // dP read them as row fragments and dQ reads K transposed, so no register
  // holds the next chunk's operands and no transpose runs on the matrix core.
  // The blocks are a static array of their own: the compiler then tells the
  // loads into them apart from every other LDS access and does not wait for
  // those loads before unrelated LDS reads and writes.
  static constexpr bool KL = KLV;
  static constexpr int KV_BYTES = 2 * HP * (D / 32) * 1024;
  static constexpr int LDS_CAP = WG_PER_CU > 0 ? 160 * 1024 / WG_PER_CU : 0;
  static constexpr bool FITS = (NW == 4 || NW == 8) && WG_PER_CU >= 1 && LDS_BYTES <= LDS_CAP &&
                               (NBIG == NW || NBIG == 4) &&
                               (!KL || (D % 32 == 0 && KC == 16 && LDS_BYTES + KV_BYTES <= LDS_CAP));
};

template <int HP, int D, int C, int KC, int HB, int FL, int NW, int WPE, bool KLV, bool ORF>
__global__ __launch_bounds__(64 * NW, WPE) void bwd_rows2_kernel(BwdParams prm) {
  using Cfg = Rows2Cfg<HP, D, C, KC, NW, WPE, KLV>;
  using ET = ETile<C, KC>;
  using DT = DTiles<D>;
  constexpr int HW = Cfg::HW, NS = Cfg::NS, NCT = Cfg::NCT, NQ = DT::NQ, RPW = Cfg::RPW, NT = 64 * NW;
  constexpr int DCW = D * C + D;
  constexpr bool KL = Cfg::KL;
  constexpr int NP = D / 32;  // 32-feature parts of a row (KL)
  extern __shared__ __align__(16) unsigned char smem[];
  bf16* Es = reinterpret_cast<bf16*>(smem);
  unsigned char* stU = smem + Cfg::E_BYTES;  // u.E, then P
  unsigned char* stW = stU + Cfg::REGION;    // w~.E + dob, then dS
  unsigned char* scal = stW + Cfg::REGION;   // increments of D
  unsigned char* scal_z = scal + 16 * 17 * 4;  // 1 / Z, after the key loop
  __shared__ __align__(16) unsigned char kv_lds[KL ? Cfg::KV_BYTES : 16];
  unsigned char* kvt = kv_lds;  // KL: [K, V][head][part] QoTile blocks of the chunk

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4, n = lane & 15;
  EventBlock eb;
  if (!tile_block(prm.ev, blockIdx.x, eb)) return;
  const int len = eb.len;
  const int H = prm.H;
  // FL >= 0: the bias flags fixed at compile time; -1: read at run time.
  const bool attn = FL >= 0 ? (FL & FST_ATTN_BIAS) != 0 : (prm.flags & FST_ATTN_BIAS) != 0;
  const bool act = FL >= 0 ? (FL & FST_ACT_BIAS) != 0 : (prm.flags & FST_ACT_BIAS) != 0;
  const bool use_e = attn || act;
  const RowAddr ra = row_addr(prm.ev, eb);   // dO, lse, D, rowsum, qt
  const RowAddr rx = row_addr_x(prm.ev, eb);  // q, k, v, dq
  const int i0 = eb.blk * 16;
  const int last = len - 1;
  bf16* dqg = reinterpret_cast<bf16*>(prm.dq);
  // The dW / db partial goes to slot blkcum[b] + tile of the work list (an
  // empty padded event owns one slot, written as zeros); tiles of padding
  // rows past an event's last tile own none.
  const int nbv = len > 0 ? (len + 15) / 16 : (prm.ev.packed ? 0 : 1);
  // The tile's slot in the work list (read once: after the prologue's
  // stores it would be read again, waiting for every load before it).
  const long tslot = (long)prm.ev.blkcum[eb.b] + eb.blk;
  float* part = eb.blk < nbv ? prm.dw_part + tslot * DCW : nullptr;
  if (event_refused(prm.ev, eb)) {
    fill_rows_nan<bf16, D>(rx, ra, i0, min(i0 + 16, len), H, tid, NT, dqg, prm.rowsum);
    if (part)
      for (int e = tid; e < DCW; e += NT) part[e] = __builtin_nanf("");
    return;
  }
  if (i0 >= len) {
    zero_tile_rows<bf16, D, NT>(prm.ev, rx, ra, i0, len, H, tid, dqg, prm.rowsum);
    if (part)
      for (int e = tid; e < DCW; e += NT) part[e] = 0.f;
    return;
  }
  const int row0 = RPW * w;  // the row-owner's first row in the tile
  // The wave's heads as head-owner: hw0 .. hw0 + nh - 1. A slot hl >= nh
  // stands for no head (the padding slot 15, past H: only where HP < 16).
  const int hw0 = w < Cfg::NBIG ? w * HW : Cfg::NBIG * HW + (w - Cfg::NBIG) * (HW - 1);
  const int nh = w < Cfg::NBIG ? HW : HW - 1;
  auto head = [&](int hl) __attribute__((always_inline)) { return hl < nh ? hw0 + hl : 15; };

  const bf16* __restrict__ qg = reinterpret_cast<const bf16*>(prm.q);
  const bf16* __restrict__ kg = reinterpret_cast<const bf16*>(prm.k);
  const bf16* __restrict__ vg = reinterpret_cast<const bf16*>(prm.v);
  const bf16* __restrict__ dog = reinterpret_cast<const bf16*>(prm.dout);
  const bf16x4 id = ident_x16(g, n);

  // The prologue issues every load it needs (the tile's q and dO, lse, W,
  // the projected rows, positions, then the first chunk's operands) before
  // its first store: a store between two loads that may alias it would make
  // the second wait for the first, one round trip per row.

  // ---- head-owner state (lane n = row i0 + n) ----
  const int my_row = i0 + n;
  const bool row_ok = my_row < len;
  KFrag<bf16, D> qf[HW], dof[HW], of[ORF ? HW : 1];
  f32x4 dQ[HW][NQ], A2[HW][NQ];
  // Dc: D - dob, the running value (ORF: the reference value until the end).
  // ORF: Nn, Zz hold this lane's parts until the end.
  float lse2[HW], Nn[HW], Zz[HW], Dc[HW];
  // Loads from a clamped row and head, without branches, so that no load
  // waits for the one before it; invalid rows and heads are zeroed below.
  const int rc = row_ok ? my_row : last;
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    const int hc = min(head(hl), H - 1);
    qf[hl].load(qg + rx.off(hc, rc, D), g);
    dof[hl].load(dog + ra.off(hc, rc, D), g);
    if constexpr (ORF) of[hl].load(reinterpret_cast<const bf16*>(prm.out) + ra.off(hc, rc, D), g);
    lse2[hl] = prm.lse[ra.vec(hc, rc)];
  }
  // ORF: the bias slots of the reference D, loaded once with the other
  // prologue loads (read after the prologue's stores, they would be loaded
  // again for every head, each time after every load before them).
  float bsl[ORF ? KFrag<bf16, D>::SLOTS : 1];
  if constexpr (ORF) {
    // Buffer loads, without branches: an empty range (no bias, or the bias
    // off) reads as zeros.
    using KF = KFrag<bf16, D>;
    const Buf bb(prm.bias, act && prm.bias ? D * 4 : 0);
#pragma unroll
    for (int t = 0; t < KF::N32; ++t)
#pragma unroll
      for (int e = 0; e < 8; e += 4) {
        const float4 v = bb.ldf4((32 * t + 8 * g + e) * 4, 0);
        bsl[8 * t + e] = v.x, bsl[8 * t + e + 1] = v.y, bsl[8 * t + e + 2] = v.z, bsl[8 * t + e + 3] = v.w;
      }
#pragma unroll
    for (int t = 0; t < KF::N16; ++t) {
      const float4 v = bb.ldf4((16 * t + 4 * g) * 4, 0);
      float* o = bsl + 8 * KF::N32 + 4 * t;
      o[0] = v.x, o[1] = v.y, o[2] = v.z, o[3] = v.w;
    }
  }

  // ---- row-owner state: rows i0 + row0 + r (r < RPW), heads on lane n ----
  WSlots<D, C> wv;
  if (use_e) wv.load(prm.weight, g, n);
  SlotRow<D> xq[RPW], xd[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int row = i0 + row0 + r;
    const bool ok = row < len && n < H;
    const int rr = row < len ? row : last;
    if (attn) xq[r].load(qg + rx.off(0, rr, D), rx.hs * D, ok, g, n);
    if (act) xd[r].load(dog + ra.off(0, rr, D), ra.hs * D, ok, g, n);
  }
  float4 pos_i = float4{0.f, 0.f, 0.f, 0.f};
  float fa[NCT], fb[NCT];
  if (use_e) {
    // Angle lanes: lane group g evaluates row row0 + g % RPW (with two rows a
    // wave, lane groups 2 and 3 repeat 0 and 1).
    const int row = i0 + row0 + g % RPW;
    pos_i = ra.pos(prm.ev.pos4, row < len ? row : last);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      fa[ct] = 1024.f * prm.freq.ghi[8 * ct + 2 * g];
      fb[ct] = 1024.f * prm.freq.ghi[8 * ct + 2 * g + 1];
    }
  }

  // ---- operand stream: K, V rows of the wave's heads, key positions ----
  const long ebase = rx.off(0, 0, D);
  const int rowb = (int)(rx.ts * D * 2);
  const unsigned ebytes = (unsigned)((prm.ev.tokmajor ? (long)len * rx.ts : (long)H * rx.hs) * D * 2);
  const Buf kbuf(kg + ebase, ebytes), vbuf(vg + ebase, ebytes);
  const Buf pbuf(prm.ev.pos4 + ra.pos_base, (unsigned)len * 16u);
  int kvo[HW];
#pragma unroll
  for (int hl = 0; hl < HW; ++hl)
    kvo[hl] = (int)(min(head(hl), H - 1) * rx.hs * D * 2) + n * rowb + kfrag_goff<D>(g);
  KFrag<bf16, D> kf[KL ? 1 : HW][NS], vf[KL ? 1 : HW][NS];
  float4 pj[NS];
  // KL: lane l of a block load fetches the quarter QoTile keeps in slot l;
  // keys past the event are clamped to its last key (their P is zero).
  const int kl_r = lane >> 2, kl_c = (lane & 3) ^ QoTile::swz(kl_r);
  // NF: chunk jn is known to be whole (no clamped keys), so its addresses
  // need no selects.
  auto issue = [&](int jn, auto nf_tag) __attribute__((always_inline)) {
    const bool full = decltype(nf_tag)::value || jn + KC <= len;
    if constexpr (KL) {
      const int rel = full ? kl_r * rowb : min(jn + kl_r, last) * rowb;
      const int soff = full ? jn * rowb : 0;
#pragma unroll
      for (int hl = 0; hl < HW; ++hl) {
        if (hl >= nh) break;
        const int h = hw0 + hl;
        const int voff = (int)(min(h, H - 1) * rx.hs * D * 2) + rel + 16 * kl_c;
#pragma unroll
        for (int t = 0; t < NP; ++t) {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(kbuf.r, (__attribute__((address_space(3))) void*)(kvt + (h * NP + t) * 1024),
                                                   16, voff + 64 * t, soff, 0, 0);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(vbuf.r, (__attribute__((address_space(3))) void*)(kvt + ((HP + h) * NP + t) * 1024),
                                                   16, voff + 64 * t, soff, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int hl = 0; hl < HW; ++hl) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const int voff = full ? kvo[hl] + 16 * s * rowb : kvo[hl] + (min(jn + 16 * s + n, last) - n) * rowb;
          const int soff = full ? jn * rowb : 0;
          load_kfrag<D>(kf[hl][s], kbuf, voff, soff);
          load_kfrag<D>(vf[hl][s], vbuf, voff, soff);
        }
      }
    }
  };
  // Key positions run one chunk further ahead: they are needed first thing
  // in a chunk.
  auto issue_pos = [&](int jn, auto nf_tag) __attribute__((always_inline)) {
    if (use_e) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        if constexpr (decltype(nf_tag)::value)
          pj[s] = pbuf.ldf4((16 * s + n) * 16, jn * 16);
        else
          pj[s] = pbuf.ldf4(min(jn + 16 * s + n, last) * 16, 0);
      }
    }
  };
  // Every chunk issues the same loads in the same order (positions, then K
  // and V; past the last chunk they reread clamped keys), so the wait at the
  // top of a chunk covers the positions only and E is formed while K and V
  // are still in flight.
  issue_pos(0, std::false_type{});
  issue(0, std::false_type{});

  // ---- prologue stores ----
  bf16* qtg = reinterpret_cast<bf16*>(prm.qt);
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    const int h = head(hl);
    const bool ok = h < H && row_ok;
    // Without branches: loads whose values a branch alone uses would be sunk
    // into it by the compiler, each then waited for with every load before it.
    qf[hl].scale_by(prm.scale);
    qf[hl].keep_if(ok);
    dof[hl].keep_if(ok);
    // Invalid rows get lse = +inf, so their P (and dS) are exactly zero.
    // (Added rather than selected: a select of the loaded value is turned
    // into a branch that the load is sunk into.)
    lse2[hl] = __builtin_fmaf(lse2[hl], kLog2e, ok ? 0.f : INFINITY);
    if (ok) {
      // qt for the cols kernel: the same bf16 values the logits use.
      bf16* qd = qtg + ra.off(h, my_row, D);
#pragma unroll
      for (int t = 0; t < KFrag<bf16, D>::N32; ++t) *reinterpret_cast<bf16x8*>(qd + 32 * t + 8 * g) = qf[hl].x32[t];
#pragma unroll
      for (int t = 0; t < KFrag<bf16, D>::N16; ++t) *reinterpret_cast<bf16x4*>(qd + 16 * t + 4 * g) = qf[hl].x16[t];
    }
    Nn[hl] = Zz[hl] = Dc[hl] = 0.f;
    if constexpr (ORF) {
      // The reference D - dob from the forward's output: dO . (out - [V] b),
      // the same sum over the keys up to the output's rounding. dS is formed
      // against it and the accumulators are corrected to N / Z once, after
      // the last chunk.
      const float part = dof[hl].dot_minus_slots(of[hl], bsl);  // 0 for invalid rows (dO zeroed)
      // Any finite reference gives the same D; a non-finite one (an output
      // that is not this forward's) falls back to 0.
      const float dref = group_allsum(part);
      Dc[hl] = __builtin_isfinite(dref) ? dref : 0.f;
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) dQ[hl][q] = A2[hl][q] = zero4();
  }
  bf16x4 uf[RPW][NCT], wf[RPW][NCT];
  f32x4 Hacc[RPW][NCT], Gacc[RPW][NCT];
  // u and w~ of the row group go to the cols kernel's scratch; rows past the
  // event are written as zeros, so every row of a group the cols kernel
  // reads is defined.
  const long uwg = tslot * 4 + (row0 >> 2);
  bf16* ug = reinterpret_cast<bf16*>(prm.u) + uwg * uw_group_elems(H, NCT);
  bf16* wtg = reinterpret_cast<bf16*>(prm.wt) + uwg * uw_group_elems(H, NCT);
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const bool ok = i0 + row0 + r < len && n < H;
    const int rg = (row0 & 3) + r;  // row within its group of four
    if (attn) {
      project_loaded<D, C>(xq[r], ok, prm.scale, wv, uf[r]);
      if (n < H)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
          *reinterpret_cast<bf16x4*>(ug + uw_off(rg >> 1, ct, n, g, rg & 1, H, NCT)) = uf[r][ct];
    }
    if (act) {
      project_loaded<D, C>(xd[r], ok, 1.f, wv, wf[r]);
      if (n < H)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
          *reinterpret_cast<bf16x4*>(wtg + uw_off(rg >> 1, ct, n, g, rg & 1, H, NCT)) = wf[r][ct];
    }
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) Hacc[r][ct] = Gacc[r][ct] = zero4();
  }

  // next_tag: the next chunk is whole (its prefetch addresses need no clamps).
  auto chunk = [&](int j0, auto tail_tag, auto next_tag) __attribute__((always_inline)) {
    constexpr bool TAIL = decltype(tail_tag)::value;
    // No prefetch past the last chunk (its loads would only hold the
    // epilogue back).
    const bool more = decltype(next_tag)::value || j0 + KC < len;
    // ---- row-owner: E, u.E and w~.E of rows row0 .. row0 + RPW - 1 ----
    if (use_e) {
      float xg[NS][4];
#pragma unroll
      for (int s = 0; s < NS; ++s) group_gather(pair_angle_unit(pos_i, pj[s]), xg[s]);
      if constexpr (!KL)
        if (more) issue_pos(j0 + KC, next_tag);
      // Each (row, subtile)'s u.E and w~.E are stored after the next one's
      // embedding is formed, which covers the products' latency.
      f32x4 ue_p = zero4(), we_p = zero4();
      int so_p = 0;
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          bf16x4 ef[NCT];
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) {
            ef[ct] = embed_step<C>(xg[s][r], fa[ct], fb[ct], ct);
            ET::store(Es, row0 + r, ct, 16 * s + n, g, ef[ct]);
          }
          if (r + s > 0) {
            if (attn) *reinterpret_cast<f32x4*>(stU + so_p) = ue_p;
            if (act) *reinterpret_cast<f32x4*>(stW + so_p) = we_p;
          }
          // Lanes of heads past HP fill padding slots nobody reads.
          so_p = stage_off(4 * s + g, row0 + r, n);
          if (attn) {
            ue_p = zero4();
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) ue_p = mfma_x16(ef[ct], uf[r][ct], ue_p);
          }
          if (act) {
            we_p = zero4();
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) we_p = mfma_x16(ef[ct], wf[r][ct], we_p);
          }
          // One (row, subtile) at a time: left free, the scheduler
          // interleaves the rows' embeddings and products into an order that
          // measured 4 % slower (likewise between head batches below).
          __builtin_amdgcn_sched_barrier(0);
        }
      if (attn) *reinterpret_cast<f32x4*>(stU + so_p) = ue_p;
      if (act) *reinterpret_cast<f32x4*>(stW + so_p) = we_p;
    }
    lds_barrier();  // u.E, w~.E staged
    // Wave priority by phase: row-owner phase 1, head-owner phase 0 (-1 %).
    __builtin_amdgcn_s_setprio(0);

    // ---- head-owner: P, dP, online D, dS, dQ (phase by phase over batches
    // of HB heads, so the heads' dependency chains overlap) ----
    // KL: this wave's K and V blocks (its own loads, issued after the
    // previous chunk's second barrier) have landed.
    if constexpr (KL) wait_vmem();
#pragma unroll
    for (int hb = 0; hb < HW; hb += HB) {
      if (hb >= nh) break;
      constexpr int NB = HB;
      f32x4 S[NB][NS], dP[NB][NS];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int hl = hb + b;
        const int h = head(hl);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          if (hl >= nh) {
            S[b][s] = dP[b][s] = zero4();
            continue;
          }
          const f32x4 ui = attn ? *reinterpret_cast<const f32x4*>(stU + stage_off(4 * s + g, n, h)) : zero4();
          const f32x4 wi = act ? *reinterpret_cast<const f32x4*>(stW + stage_off(4 * s + g, n, h)) : zero4();
          if constexpr (KL) {
            KFrag<bf16, D> kc, vc;
#pragma unroll
            for (int t = 0; t < NP; ++t) {
              kc.x32[t] = QoTile::row_frag(kvt + (h * NP + t) * 1024, g, n);
              vc.x32[t] = QoTile::row_frag(kvt + ((HP + h) * NP + t) * 1024, g, n);
            }
            S[b][s] = mma_k<D>(kc, qf[hl], ui);
            dP[b][s] = mma_k<D>(vc, dof[hl], wi);
          } else {
            S[b][s] = mma_k<D>(kf[hl][s], qf[hl], ui);
            dP[b][s] = mma_k<D>(vf[hl][s], dof[hl], wi);
          }
        }
      }
      float nt[NB], zt[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int hl = hb + b < HW ? hb + b : HW - 1;
        float a = ORF ? Nn[hl] : -0.f, z = ORF ? Zz[hl] : -0.f;
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float p = exp2f_fast(__builtin_fmaf(S[b][s][r], kLog2e, -lse2[hl]));
            if constexpr (TAIL) p = (j0 + 16 * s + 4 * g + r < len) ? p : 0.f;
            S[b][s][r] = p;
            a = __builtin_fmaf(p, dP[b][s][r], a);
            z += p;
          }
        nt[b] = a;
        zt[b] = z;
      }
      float dD[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int hl = hb + b;
        if (hl >= nh) continue;
        if constexpr (ORF) {
          Nn[hl] = nt[b];
          Zz[hl] = zt[b];
          dD[b] = 0.f;
        } else {
          group_allsum2(nt[b], zt[b]);
          Nn[hl] += nt[b];
          Zz[hl] += zt[b];
          const float dn = Zz[hl] > 0.f ? Nn[hl] * __builtin_amdgcn_rcpf(Zz[hl]) : 0.f;
          dD[b] = dn - Dc[hl];
          Dc[hl] = dn;
        }
      }
      JFrag<bf16, NS> pf[NB], dsf[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int hl = hb + b;
        if (hl >= nh) continue;
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) dP[b][s][r] = S[b][s][r] * (dP[b][s][r] - Dc[hl]);
        pf[b].from_tiles(S[b]);
        dsf[b].from_tiles(dP[b]);
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int hl = hb + b;
        if (hl >= nh) continue;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          JFrag<bf16, NS> kt;
          if constexpr (KL)
            kt.v = QoTile::tr_frag_dmap(kvt + (head(hl) * NP + (q >> 1)) * 1024, q, g, n);
          else if constexpr (NS == 2)
            kt.v = cat8(transpose_x16(DT::part(kf[hl][0], q), id), transpose_x16(DT::part(kf[hl][1], q), id));
          else
            kt.v = transpose_x16(DT::part(kf[hl][0], q), id);
          if constexpr (!ORF) dQ[hl][q] = dQ[hl][q] - dD[b] * A2[hl][q];
          A2[hl][q] = mma_j(kt, pf[b], A2[hl][q]);
          dQ[hl][q] = mma_j(kt, dsf[b], dQ[hl][q]);
        }
      }
      if (use_e) {
        // P and dS for the row-owner (keys 16s + 4g .. +3 of slot (row n,
        // head h)), and the increment of D.
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int hl = hb + b;
          const int h = head(hl);
          if (hl >= nh) continue;
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            bf16x4 pv, dv;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              pv[r] = pf[b].v[4 * s + r];
              dv[r] = dsf[b].v[4 * s + r];
            }
            const int so = half_off(2 * s + (g >> 1), n, h, g & 1);
            *reinterpret_cast<bf16x4*>(stU + so) = pv;
            *reinterpret_cast<bf16x4*>(stW + so) = dv;
          }
          if constexpr (!ORF) *reinterpret_cast<float*>(scal + scal_off(n, h)) = dD[b];  // the same value from every lane group
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (!KL)
      if (more) issue(j0 + KC, next_tag);
    __builtin_amdgcn_s_setprio(1);
    lds_barrier();  // P, dS and D increments staged
    // KL: the next chunk's positions go out here, its K and V loads at the
    // end of the chunk: every transposing LDS read the compiler cannot tell
    // apart from their destination (the E reads below) waits for loads into
    // LDS in flight.
    if constexpr (KL)
      if (more) issue_pos(j0 + KC, next_tag);

    // ---- row-owner: H -= dD G; H += E^T dS; G += E^T P ----
    if (use_e) {
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const int il = row0 + r;
        // Lanes of padded heads (n >= H) read some other slot of the row:
        // finite values whose columns of H and G are never used.
        const int hn = n < HP ? n : HP - 1;
        const float dd = ORF ? 0.f : *reinterpret_cast<const float*>(scal + scal_off(il, n));
        JFrag<bf16, NS> pr, dr;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const int so = half_off(2 * s + (g >> 1), il, hn, g & 1);
          const bf16x4 pv = *reinterpret_cast<const bf16x4*>(stU + so);
          const bf16x4 dv = *reinterpret_cast<const bf16x4*>(stW + so);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pr.v[4 * s + e] = pv[e];
            dr.v[4 * s + e] = dv[e];
          }
        }
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
          JFrag<bf16, NS> et;
          if constexpr (NS == 2)
            et.v = cat8(ET::load_tr(Es, il, ct, 0, g, n), ET::load_tr(Es, il, ct, 16, g, n));
          else
            et.v = ET::load_tr(Es, il, ct, 0, g, n);
          if (attn) {
            if constexpr (!ORF) Hacc[r][ct] = Hacc[r][ct] - dd * Gacc[r][ct];
            Hacc[r][ct] = mma_j(et, dr, Hacc[r][ct]);
          }
          Gacc[r][ct] = mma_j(et, pr, Gacc[r][ct]);
        }
      }
    }
    if constexpr (KL)
      if (more) issue(j0 + KC, next_tag);
  };

  int j0 = 0;
  for (; j0 + 2 * KC <= len; j0 += KC) chunk(j0, std::false_type{}, std::true_type{});
  if (j0 + KC <= len) {
    chunk(j0, std::false_type{}, std::false_type{});
    j0 += KC;
  }
  if (j0 < len) chunk(j0, std::true_type{}, std::false_type{});
  // KL: the loads of the chunk past the last finish before the workgroup
  // ends.
  if constexpr (KL) wait_vmem();

  // D = N / Z over all keys. ORF: dQ and H, built against the reference
  // value, take the P sums they lack: dQ -= (D - Dref) sum P k, H -= (D -
  // Dref) G. Then every accumulator is divided by Z: P = exp(s - lse) with
  // the forward's rounded lse carries a common factor per row (Z = sum P
  // = 1 up to that rounding, ~1e-3 off at logits of O(1e4)), which P / Z
  // removes; the cols kernel recomputes P / Z from lse_z.
  float dD[HW], rz[HW];
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    if constexpr (ORF) {
      group_allsum2(Nn[hl], Zz[hl]);
      const float dn = Zz[hl] > 0.f ? Nn[hl] * __builtin_amdgcn_rcpf(Zz[hl]) : 0.f;
      dD[hl] = dn - Dc[hl];
      Dc[hl] = dn;
#pragma unroll
      for (int q = 0; q < NQ; ++q) dQ[hl][q] = dQ[hl][q] - dD[hl] * A2[hl][q];
    }
    rz[hl] = Zz[hl] > 0.f ? 1.f / Zz[hl] : 1.f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) dQ[hl][q] = dQ[hl][q] * rz[hl];
  }
  if (use_e) {
#pragma unroll
    for (int hl = 0; hl < HW; ++hl)
      if (hl < nh) {
        if (ORF && attn) *reinterpret_cast<float*>(scal + scal_off(n, head(hl))) = dD[hl];
        *reinterpret_cast<float*>(scal_z + scal_off(n, head(hl))) = rz[hl];
      }
    __syncthreads();
    // Lanes of padded heads (n >= HP) read some other slot: finite values in
    // columns of H and G that are never used.
    const int hn = n < HP ? n : HP - 1;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const float zr = *reinterpret_cast<const float*>(scal_z + scal_off(row0 + r, hn));
      if (ORF && attn) {
        const float dd = *reinterpret_cast<const float*>(scal + scal_off(row0 + r, hn));
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) Hacc[r][ct] = Hacc[r][ct] - dd * Gacc[r][ct];
      }
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        Hacc[r][ct] = Hacc[r][ct] * zr;
        Gacc[r][ct] = Gacc[r][ct] * zr;
      }
    }
  }

  // ---- epilogue: sigma, D, dq = scale (dQ + W H + sigma b) ----
  // W (d on the lanes, the slots of H on the k index) as bf16 parts, and b,
  // loaded before the first barrier.
  bf16x4 wdh[NQ][NCT], wdl[NQ][NCT];
  float bq[NQ][4];
  if (attn) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int dn = DT::dmap(q, n >> 2, n & 3);
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        f32x4 wq;
#pragma unroll
        for (int sp = 0; sp < 4; ++sp) wq[sp] = prm.weight[dn * C + slot_channel<C>(16 * ct + 4 * g + sp)];
        split4(wq, wdh[q][ct], wdl[q][ct]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) bq[q][r] = prm.bias ? prm.bias[DT::dmap(q, g, r)] : 0.f;
    }
  }
  float sig[HW];
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    sig[hl] = (Nn[hl] - Dc[hl] * Zz[hl]) * rz[hl];
    const int h = head(hl);
    if (g == 0 && row_ok && h < H) {
      prm.dsum[ra.vec(h, my_row)] = Dc[hl];  // D - dob: the cols kernel's dS = P (dP~ - (D - dob))
      // The cols kernel's exponent offset: its P is exp2(s log2 e - lse_z) = P / Z.
      prm.lse_z[ra.vec(h, my_row)] = lse2[hl] + (Zz[hl] > 0.f ? __builtin_amdgcn_logf(Zz[hl]) : 0.f);
      if (prm.rowsum) prm.rowsum[ra.vec(h, my_row)] = sig[hl];
    }
  }
  // W H on bf16 MFMA over the two parts of each factor (W and H to 16 bits).
  bf16x4 hh[RPW][NCT], hlo[RPW][NCT];
  if (attn) {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) split4(Hacc[r][ct], hh[r][ct], hlo[r][ct]);
  }
  // Two head-dim tiles per exchange, staged in the u.E and w~.E regions.
  constexpr int QR = NQ >= 2 ? 2 : 1;
#pragma unroll
  for (int q0 = 0; q0 < NQ; q0 += QR) {
    if (attn) {
      __syncthreads();  // the stage is free (last chunk, or previous round)
#pragma unroll
      for (int qq = 0; qq < QR; ++qq) {
        const int q = q0 + qq;
        if (q >= NQ) break;
        unsigned char* st = qq == 0 ? stU : stW;
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          f32x4 acc = zero4();
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) acc = mma_split(wdh[q][ct], wdl[q][ct], hh[r][ct], hlo[r][ct], acc);
          *reinterpret_cast<f32x4*>(st + stage_off(g, row0 + r, n)) = acc;
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int qq = 0; qq < QR; ++qq) {
      const int q = q0 + qq;
      if (q >= NQ) break;
      const unsigned char* st = qq == 0 ? stU : stW;
#pragma unroll
      for (int hl = 0; hl < HW; ++hl) {
        const int h = head(hl);
        f32x4 o = dQ[hl][q];
        if (attn && h < H) {
          o = o + *reinterpret_cast<const f32x4*>(st + stage_off(g, n, h));
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = __builtin_fmaf(sig[hl], bq[q][r], o[r]);
        }
        dQ[hl][q] = o * prm.scale;
      }
    }
  }
  if (row_ok) {
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
      const int h = head(hl);
      if (h >= H) continue;
      bf16* orow = dqg + rx.off(h, my_row, D);
      if constexpr (DT::X32) {
#pragma unroll
        for (int t = 0; t < NQ / 2; ++t)
          *reinterpret_cast<bf16x8*>(orow + DT::dmap(2 * t, g, 0)) =
              cat8(pack4(dQ[hl][2 * t]), pack4(dQ[hl][2 * t + 1]));
      } else {
#pragma unroll
        for (int q = 0; q < NQ; ++q) *reinterpret_cast<bf16x4*>(orow + DT::dmap(q, g, 0)) = pack4(dQ[hl][q]);
      }
    }
  }

  // ---- dW / db partial of this tile: sum over its rows and heads ----
  // dW[d, channel(slot)] += sum_(row, head) A[d, (row, head)] B[(row, head), slot]
  // on bf16 MFMA, each wave over its own rows: A = qt (then dO) with d on the
  // lanes, read from the tile's rows that the head-owners stage ([op][row]
  // [head][D], zeros for invalid rows and heads: the one exchange between
  // waves); B = H (then G) with the slot on the lanes, which the wave stages
  // for itself one channel step at a time as [row][head][16 slots].
  __syncthreads();
  float* Wred = reinterpret_cast<float*>(smem);  // after the products, over Xs
  bf16* Xs = reinterpret_cast<bf16*>(smem);
  float* HGs = reinterpret_cast<float*>(smem + Cfg::X_DW);
  if (use_e) {
    f32x4 dw[NQ][NCT];
    float dbl[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      dbl[q] = 0.f;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) dw[q][ct] = zero4();
    }
#pragma unroll
    for (int op = 0; op < 2; ++op) {
      if (!(op == 0 ? attn : act)) continue;
#pragma unroll
      for (int hl = 0; hl < HW; ++hl) {
        const int h = head(hl);
        if (h < HP) (op == 0 ? qf[hl] : dof[hl]).store(Xs + (op * HP + h) * Cfg::XS_HS + n * Cfg::XS_RS, g);
      }
    }
    __syncthreads();
#pragma unroll
    for (int op = 0; op < 2; ++op) {
      if (!(op == 0 ? attn : act)) continue;
      const bf16* Xo = Xs + op * HP * Cfg::XS_HS;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        // The wave's own rows, exchanged between its lanes: wave_lds_sync
        // (a compiler fence and an LDS wait) orders the stores after the
        // previous step's reads and before this step's, in place of a
        // workgroup barrier.
        wave_lds_sync();
#pragma unroll
        for (int r = 0; r < RPW; ++r)
          if (n < HP)
            *reinterpret_cast<f32x4*>(HGs + ((row0 + r) * HP + n) * 16 + 4 * g) = op == 0 ? Hacc[r][ct] : Gacc[r][ct];
        wave_lds_sync();
        // One 16x16x16 product per head quad s4: k-slot 4g + e is the pair
        // (row row0 + e, head 4 s4 + g) (e < RPW; the rest zero), A = the
        // staged bf16 rows (exact), B = H or G in two bf16 parts.
#pragma unroll
        for (int s4 = 0; s4 < HP / 4; ++s4) {
          const int h = 4 * s4 + g;
          f32x4 bv = zero4();
#pragma unroll
          for (int e = 0; e < RPW && e < 4; ++e) bv[e] = HGs[((row0 + e) * HP + h) * 16 + n];
          bf16x4 bh, bl;
          split4(bv, bh, bl);
#pragma unroll
          for (int q = 0; q < NQ; ++q) {
            // Lane n of the group receives rows row0 .. row0 + 3 of feature
            // 16 q + n; source lane n supplies row row0 + n / 4 (clamped to
            // the wave's rows: the others meet zero slots of B), features
            // 16 q + 4 (n % 4) .. + 3.
            const bf16* src = Xo + h * Cfg::XS_HS + (row0 + min(n >> 2, RPW - 1)) * Cfg::XS_RS + 16 * q + 4 * (n & 3);
            const bf16x4 av = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(src));
            if (op == 1 && ct == 0)
#pragma unroll
              for (int e = 0; e < RPW && e < 4; ++e) dbl[q] += (float)av[e];
            dw[q][ct] = mfma_x16(av, bl, dw[q][ct]);
            dw[q][ct] = mfma_x16(av, bh, dw[q][ct]);
          }
        }
      }
    }
    __syncthreads();  // every wave done with Xs before the partials overwrite it
    // Four partials: wave w's (w < 4), then with eight waves wave w + 4's
    // added to slot w in a second round (a fixed order of additions).
    float* wr = Wred + (w & 3) * DCW;
    float dbs[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) dbs[q] = group_allsum(dbl[q]);
#pragma unroll
    for (int round = 0; round < NW / 4; ++round) {
      if (round > 0) __syncthreads();
      if ((w >> 2) == round) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float& slot = wr[(16 * q + 4 * g + r) * C + slot_channel<C>(16 * ct + n)];
              slot = round > 0 ? slot + dw[q][ct][r] : dw[q][ct][r];
            }
          if (g == 0) wr[D * C + 16 * q + n] = round > 0 ? wr[D * C + 16 * q + n] + dbs[q] : dbs[q];
        }
      }
    }
    __syncthreads();
    for (int e = tid; e < DCW; e += NT) part[e] = Wred[e] + Wred[DCW + e] + Wred[2 * DCW + e] + Wred[3 * DCW + e];
  } else {
    for (int e = tid; e < DCW; e += NT) part[e] = 0.f;
  }

  zero_tile_rows<bf16, D, NT>(prm.ev, rx, ra, i0, len, H, tid, dqg, prm.rowsum);
}

// ---------------------------------------------------------------------------
// Cols kernel.
// ---------------------------------------------------------------------------
template <int HP, int D, int C, int RC>
struct Cols2Cfg {
  static constexpr int HW = HP / 4, NS = RC / 16, NCT = C / 16;
  static constexpr int RG = RC / 4;     // row groups per chunk
  static constexpr int RGW = RC / 16;   // row groups per row-owner wave
  static constexpr int REGION = RG * HP * 16 * 16;  // one fp32 term: [row group][HP heads][key] x 4 rows
  static constexpr int SCAL_BYTES = 2 * RC * 16 * 4;  // lse * log2(e) and D - dob: [term][head][row]
  static constexpr int BASE_BYTES = 2 * REGION + SCAL_BYTES;
  // QL: the chunk's qt and dO rows are staged in LDS (QoTile), so both their
  // row-major and transposed operand fragments are LDS reads; otherwise they
  // stream through registers and are transposed on the matrix core.
  static constexpr int QO_BYTES = 2 * HP * (D / 32) * 1024;
  static constexpr bool QL = D % 32 == 0 && RC == 16 && BASE_BYTES + QO_BYTES <= 80 * 1024;
  static constexpr int LDS_BYTES = BASE_BYTES + (QL ? QO_BYTES : 0);
  static constexpr bool FITS = LDS_BYTES <= 80 * 1024 && HP % 4 == 0;
};


template <int HP, int D, int C, int RC, int FL, int OCC>
__global__ __launch_bounds__(256, OCC) void bwd_cols2_kernel(BwdParams prm) {
  using Cfg = Cols2Cfg<HP, D, C, RC>;
  using DT = DTiles<D>;
  constexpr int HW = Cfg::HW, NS = Cfg::NS, NCT = Cfg::NCT, NQ = DT::NQ, RGW = Cfg::RGW;
  constexpr bool QL = Cfg::QL;
  // TR: the transposed qt / dO reads in QoTile::tr_frag's order, free of
  // bank conflicts, with dk / dv regathered into 16-byte store order through
  // LDS once per tile; elsewhere tr_frag_dmap's order, which needs no
  // regather. Measured (bitwise equal): D = C = 64 with HP <= 8 cols -1.7 to
  // -5 % (cfg4 3.15 -> 3.02 ms; H = 4 -2.4 %); C = 32 or 48, HP = 12 or
  // D = 32 +0.6 to +6 %, so only there.
  constexpr bool TR = QL && D == 64 && C == 64 && HP <= 8;
  constexpr int NP = D / 32;  // 32-feature parts of a row (QL)
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* stU = smem;                 // u.E
  unsigned char* stW = smem + Cfg::REGION;   // w~.E
  float* rsc = reinterpret_cast<float*>(smem + 2 * Cfg::REGION);  // per-row scalars of the chunk
  unsigned char* qo = smem + Cfg::BASE_BYTES;  // QL: [qt, dO][head][part] QoTile blocks

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4, n = lane & 15;

  EventSpec ev = prm.ev;
  ev.blkcum = prm.blkcum_cols;
  ev.scum = prm.scum_cols;
  ev.vp = nullptr;  // the interleaved schedule (the padding-last one is the rows kernel's)
  EventBlock eb;
  if (!tile_block(ev, blockIdx.x, eb)) return;
  const int len = eb.len;
  const int H = prm.H;
  // FL >= 0: the bias flags fixed at compile time; -1: read at run time.
  const bool attn = FL >= 0 ? (FL & FST_ATTN_BIAS) != 0 : (prm.flags & FST_ATTN_BIAS) != 0;
  const bool act = FL >= 0 ? (FL & FST_ACT_BIAS) != 0 : (prm.flags & FST_ACT_BIAS) != 0;
  const bool use_e = attn || act;
  const RowAddr ra = row_addr(ev, eb);   // qt, dO, lse, D
  const RowAddr rx = row_addr_x(ev, eb);  // k, v, dk, dv
  const int k0 = eb.blk * 16;
  const int last = len - 1;
  bf16* dkg = reinterpret_cast<bf16*>(prm.dk);
  bf16* dvg = reinterpret_cast<bf16*>(prm.dv);
  if (event_refused(ev, eb)) {
    fill_rows_nan<bf16, D>(rx, rx, k0, min(k0 + 16, len), H, tid, 256, dkg, nullptr);
    fill_rows_nan<bf16, D>(rx, rx, k0, min(k0 + 16, len), H, tid, 256, dvg, nullptr);
    return;
  }
  if (k0 >= len) {
    zero_tile_rows<bf16, D>(ev, rx, rx, k0, len, H, tid, dkg, nullptr);
    zero_tile_rows<bf16, D>(ev, rx, rx, k0, len, H, tid, dvg, nullptr);
    return;
  }
  const bf16x4 id = ident_x16(g, n);

  // ---- head-owner state (lane n = key k0 + n) ----
  const int my_key = k0 + n;
  const bool key_ok = my_key < len;
  const int kc = key_ok ? my_key : last;
  KFrag<bf16, D> kf[HW], vf[HW];
  f32x4 dK[HW][NQ], dV[HW][NQ];
  const bf16* __restrict__ kg = reinterpret_cast<const bf16*>(prm.k);
  const bf16* __restrict__ vg = reinterpret_cast<const bf16*>(prm.v);
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    // Padded heads (h >= H) compute on head H-1's data and are never stored.
    const int hq = min(w * HW + hl, H - 1);
    kf[hl].load(kg + rx.off(hq, kc, D), g);
    vf[hl].load(vg + rx.off(hq, kc, D), g);
#pragma unroll
    for (int q = 0; q < NQ; ++q) dK[hl][q] = dV[hl][q] = zero4();
  }

  // ---- row-owner: streamed rows 4 (RGW w + q') + r of each chunk ----
  float4 pos_k = float4{0.f, 0.f, 0.f, 0.f};
  float fa[NCT], fb[NCT];
  if (use_e) {
    pos_k = ra.pos(ev.pos4, kc);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      fa[ct] = 1024.f * prm.freq.ghi[8 * ct + 2 * g];
      fb[ct] = 1024.f * prm.freq.ghi[8 * ct + 2 * g + 1];
    }
  }

  // ---- operand stream: qt and dO rows of the wave's heads, per-row scalars,
  // u / w~ rows and row positions ----
  const long ebase = ra.off(0, 0, D);
  const int rowb = (int)(ra.ts * D * 2);
  const unsigned ebytes = (unsigned)((ev.tokmajor ? (long)len * ra.ts : (long)H * ra.hs) * D * 2);
  const Buf qbuf(reinterpret_cast<const bf16*>(prm.qt) + ebase, ebytes);
  const Buf obuf(reinterpret_cast<const bf16*>(prm.dout) + ebase, ebytes);
  const unsigned vbytes = (unsigned)((ev.tokmajor ? (long)len * ra.ts : (long)H * ra.hs) * 4);
  const Buf lbuf(prm.lse_z + ra.base_row, vbytes), dbuf(prm.dsum + ra.base_row, vbytes);
  // u / w~ in the row-group layout the rows kernel writes (uw_off): the
  // event's groups start at 4 x its first tile in the rows work list.
  const long ggrp = uw_group_elems(H, NCT);
  const long cbase = (long)prm.ev.blkcum[eb.b] * 4 * ggrp;
  const int glast = (len - 1) >> 2;  // last row group of the event
  const unsigned cbytes = (unsigned)((long)(glast + 1) * ggrp * 2);
  const Buf ubuf(reinterpret_cast<const bf16*>(prm.u) + cbase, cbytes),
      wbuf(reinterpret_cast<const bf16*>(prm.wt) + cbase, cbytes);
  const Buf pbuf(ev.pos4 + ra.pos_base, (unsigned)len * 16u);
  int qvo[HW];
#pragma unroll
  for (int hl = 0; hl < HW; ++hl)
    qvo[hl] = (int)(min(w * HW + hl, H - 1) * ra.hs * D * 2) + n * rowb + kfrag_goff<D>(g);

  KFrag<bf16, D> qr[QL ? 1 : HW][NS], orw[QL ? 1 : HW][NS];
  // Per-row scalars (the rows kernel's lse_z = lse log2 e + log2 Z, so that
  // P = exp2(s log2 e - lse_z) is normalised, and D - dob) of the next chunk: thread t
  // loads item t of the chunk's RC x H values of each (coalesced), and writes
  // it to LDS at the start of that chunk; the head-owners read four rows at a
  // time (one 16-byte broadcast read).
  // The raw values are kept until the chunk's scalars are written, so the
  // loads are not waited for where they are issued.
  float sc_lraw = 0.f, sc_draw = 0.f;
  const int sc_h = ev.tokmajor ? tid % H : tid / RC;
  const int sc_r = ev.tokmajor ? tid / H : tid % RC;
  const bool sc_ok = tid < RC * H;
  const int sc_hc = min(sc_h, H - 1);
  float4 prow[RGW];
  // QL: the wave's heads' qt and dO rows of a chunk go straight to LDS, lane
  // l of a block load fetching the quarter QoTile keeps in slot l; rows past
  // the event are clamped to its last row.
  const int qo_r = lane >> 2, qo_c = (lane & 3) ^ QoTile::swz(qo_r);
  auto issue_qo = [&](int in) __attribute__((always_inline)) {
    if constexpr (QL) {
      const bool full = in + RC <= len;
      const int rel = full ? qo_r * rowb : (min(in + qo_r, last)) * rowb;
      const int soff = full ? in * rowb : 0;
#pragma unroll
      for (int hl = 0; hl < HW; ++hl) {
        const int h = w * HW + hl;
        const int voff = (int)(min(h, H - 1) * ra.hs * D * 2) + rel + 16 * qo_c;
#pragma unroll
        for (int t = 0; t < NP; ++t) {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(qbuf.r, (__attribute__((address_space(3))) void*)(qo + ((0 * HP + h) * NP + t) * 1024),
                                                   16, voff + 64 * t, soff, 0, 0);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(obuf.r, (__attribute__((address_space(3))) void*)(qo + ((1 * HP + h) * NP + t) * 1024),
                                                   16, voff + 64 * t, soff, 0, 0);
        }
      }
    }
  };
  // NF: chunk `in` is known to be whole (no clamped rows), so its addresses
  // need no selects or clamps.
  auto issue = [&](int in, auto nf_tag) __attribute__((always_inline)) {
    constexpr bool NF = decltype(nf_tag)::value;
    if constexpr (!QL) {
      const bool full = NF || in + RC <= len;
#pragma unroll
      for (int hl = 0; hl < HW; ++hl) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const int voff = full ? qvo[hl] + 16 * s * rowb : qvo[hl] + (min(in + 16 * s + n, last) - n) * rowb;
          const int soff = full ? in * rowb : 0;
          load_kfrag<D>(qr[hl][s], qbuf, voff, soff);
          load_kfrag<D>(orw[hl][s], obuf, voff, soff);
        }
      }
    }
    if constexpr (NF) {
      const int vo = (int)(sc_hc * ra.hs + sc_r * ra.ts) * 4, so = (int)(in * ra.ts) * 4;
      sc_lraw = lbuf.ldf(vo, so);
      sc_draw = dbuf.ldf(vo, so);
    } else {
      const int vo = (int)(ra.vec(sc_hc, min(in + sc_r, last)) - ra.base_row) * 4;
      sc_lraw = lbuf.ldf(vo, 0);
      sc_draw = dbuf.ldf(vo, 0);
    }
  };
  // Row positions and the u / w~ rows of the row-owner part run one chunk
  // further ahead: they are needed first thing in a chunk.
  bf16x4 ur[RGW][4][NCT], wr[RGW][4][NCT];
  auto issue_rows = [&](int in, auto nf_tag) __attribute__((always_inline)) {
    constexpr bool NF = decltype(nf_tag)::value;
    if (use_e) {
#pragma unroll
      for (int q2 = 0; q2 < RGW; ++q2) {
        const int rg = RGW * w + q2;
        if constexpr (NF)
          prow[q2] = pbuf.ldf4((4 * rg + g) * 16, in * 16);
        else
          prow[q2] = pbuf.ldf4(min(in + 4 * rg + g, last) * 16, 0);
        // Groups past the event reread its last group: their rows carry
        // P = 0 (lse = +inf) in the head-owner part.
        const int go = NF ? (int)(rg * ggrp) : (int)(min((in >> 2) + rg, glast) * ggrp);
        const int gso = NF ? (int)((in >> 2) * ggrp) * 2 : 0;
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) {
            const int co = (go + uw_off(half, ct, n, g, 0, H, NCT)) * 2;
            if (attn) {
              const bf16x8 v = ubuf.ld128(co, gso);
              ur[q2][2 * half][ct] = lo4(v);
              ur[q2][2 * half + 1][ct] = hi4(v);
            }
            if (act) {
              const bf16x8 v = wbuf.ld128(co, gso);
              wr[q2][2 * half][ct] = lo4(v);
              wr[q2][2 * half + 1][ct] = hi4(v);
            }
          }
      }
    }
  };
  // Every chunk issues the same loads in the same order (the row-owner's
  // rows, then the head-owner's; past the last chunk they reread clamped
  // rows), so each phase waits only for the loads it uses.
  issue_rows(0, std::false_type{});
  issue(0, std::false_type{});

  // next_tag: the next chunk is whole (its prefetch addresses need no clamps).
  auto chunk = [&](int i0c, auto tail_tag, auto next_tag) __attribute__((always_inline)) {
    constexpr bool TAIL = decltype(tail_tag)::value;
    // No prefetch past the last chunk (its loads would only hold the
    // epilogue back).
    const bool more = decltype(next_tag)::value || i0c + RC < len;
    issue_qo(i0c);  // lands during the row-owner part
    // ---- row-owner: u_i E_i^T and w~_i E_i^T for its row groups ----
    if (use_e) {
#pragma unroll
      for (int q2 = 0; q2 < RGW; ++q2) {
        const int rg = RGW * w + q2;
        float xg[4];
        group_gather(pair_angle_unit(prow[q2], pos_k), xg);
        f32x4 ue[4], we[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          bf16x4 ef[NCT];
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) ef[ct] = embed_step<C>(xg[r], fa[ct], fb[ct], ct);
          ue[r] = we[r] = zero4();
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) {
            if (attn) ue[r] = mfma_x16(ur[q2][r][ct], ef[ct], ue[r]);
            if (act) we[r] = mfma_x16(wr[q2][r][ct], ef[ct], we[r]);
          }
        }
        // lane (g, key n) holds heads 4g + e of rows r: regroup by head.
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // Heads past HP (lane groups g >= HP / 4) have no slot.
          const int so = ((rg * HP + 4 * g + e) * 16 + n) * 16;
          if (4 * g < HP) {
            if (attn) *reinterpret_cast<f32x4*>(stU + so) = f32x4{ue[0][e], ue[1][e], ue[2][e], ue[3][e]};
            if (act) *reinterpret_cast<f32x4*>(stW + so) = f32x4{we[0][e], we[1][e], we[2][e], we[3][e]};
          }
        }
      }
    }
    if constexpr (!QL)
      if (more) issue_rows(i0c + RC, next_tag);
    if (sc_ok) {
      rsc[sc_h * RC + sc_r] = i0c + sc_r < len ? sc_lraw : INFINITY;  // rows past the event: P = 0
      rsc[16 * RC + sc_h * RC + sc_r] = sc_draw;
    }
    lds_barrier();  // u.E, w~.E and the row scalars staged
    // Wave priority by phase: head-owner phase 1, row-owner phase 0 (-1.7 %).
    __builtin_amdgcn_s_setprio(1);
    // QL: this wave's own direct-to-LDS qt / dO rows (read by it alone) have
    // landed; waited for after the barrier, before the next rows' loads.
    if constexpr (QL) wait_vmem();
    if constexpr (QL)
      if (more) issue_rows(i0c + RC, next_tag);

    // ---- head-owner: P, dS, dV^T += dO^T P, dK^T += Qt^T dS ----
    f32x4 S[HW][NS], dP[HW][NS];
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
      const int h = w * HW + hl;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int so = (((4 * s + g) * HP + h) * 16 + n) * 16;
        const f32x4 ui = attn ? *reinterpret_cast<const f32x4*>(stU + so) : zero4();
        const f32x4 wi = act ? *reinterpret_cast<const f32x4*>(stW + so) : zero4();
        if constexpr (QL) {
          KFrag<bf16, D> qf, of;
#pragma unroll
          for (int t = 0; t < NP; ++t) {
            qf.x32[t] = QoTile::row_frag(qo + ((0 * HP + h) * NP + t) * 1024, g, n);
            of.x32[t] = QoTile::row_frag(qo + ((1 * HP + h) * NP + t) * 1024, g, n);
          }
          S[hl][s] = mma_k<D>(qf, kf[hl], ui);
          dP[hl][s] = mma_k<D>(of, vf[hl], wi);
        } else {
          S[hl][s] = mma_k<D>(qr[hl][s], kf[hl], ui);
          dP[hl][s] = mma_k<D>(orw[hl][s], vf[hl], wi);
        }
      }
    }
    JFrag<bf16, NS> pf[HW], dsf[HW];
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
      const int h = min(w * HW + hl, H - 1);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const f32x4 lse2 = *reinterpret_cast<const f32x4*>(rsc + h * RC + 16 * s + 4 * g);
        const f32x4 dsv = *reinterpret_cast<const f32x4*>(rsc + 16 * RC + h * RC + 16 * s + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // Rows past the event carry lse = +inf: P = 0 there.
          const float p = exp2f_fast(__builtin_fmaf(S[hl][s][r], kLog2e, -lse2[r]));
          S[hl][s][r] = p;
          dP[hl][s][r] = p * (dP[hl][s][r] - dsv[r]);
        }
      }
      pf[hl].from_tiles(S[hl]);
      dsf[hl].from_tiles(dP[hl]);
      // One head's P and dS at a time where a wave owns three heads or more
      // and D <= 48, and at D = 48 (H = 12, D = 32: 2-3 % faster than the
      // scheduler's own interleaving of the heads; H = 8, D = 48: 0-2 %; at
      // D = 64 it measured 18-21 % slower, and 3 % slower at two heads of
      // D = 32).
      if constexpr ((HW >= 3 && D <= 48) || D == 48) __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        JFrag<bf16, NS> ot, qt;
        if constexpr (QL) {
          const int h = w * HW + hl;
          const unsigned char* ob = qo + ((1 * HP + h) * NP + (q >> 1)) * 1024;
          const unsigned char* qb = qo + ((0 * HP + h) * NP + (q >> 1)) * 1024;
          ot.v = TR ? QoTile::tr_frag(ob, q, g, n) : QoTile::tr_frag_dmap(ob, q, g, n);
          qt.v = TR ? QoTile::tr_frag(qb, q, g, n) : QoTile::tr_frag_dmap(qb, q, g, n);
        } else if constexpr (NS == 2) {
          ot.v = cat8(transpose_x16(DT::part(orw[hl][0], q), id), transpose_x16(DT::part(orw[hl][1], q), id));
          qt.v = cat8(transpose_x16(DT::part(qr[hl][0], q), id), transpose_x16(DT::part(qr[hl][1], q), id));
        } else {
          ot.v = transpose_x16(DT::part(orw[hl][0], q), id);
          qt.v = transpose_x16(DT::part(qr[hl][0], q), id);
        }
        dV[hl][q] = mma_j(ot, pf[hl], dV[hl][q]);
        dK[hl][q] = mma_j(qt, dsf[hl], dK[hl][q]);
      }
    }
    (void)TAIL;
    if (more) issue(i0c + RC, next_tag);
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();  // the stage is read; the next chunk may overwrite it
  };

  int i0c = 0;
  for (; i0c + 2 * RC <= len; i0c += RC) chunk(i0c, std::false_type{}, std::true_type{});
  if (i0c + RC <= len) {
    chunk(i0c, std::false_type{}, std::false_type{});
    i0c += RC;
  }
  if (i0c < len) chunk(i0c, std::true_type{}, std::false_type{});

  // ---- store dk, dv (lane n = key) ----
  // Accumulator q holds features DTiles::dmap(q, g, r) (with the tiles in LDS
  // (QL) the transposed reads' order), or under TR 16 q + 4 g + r, regathered
  // into dmap order first: where D is a multiple of 32, 8 consecutive
  // features per lane group across the accumulator pair 2t, 2t + 1.
  [[maybe_unused]] bf16x8 kst[HW][NQ / 2 > 0 ? NQ / 2 : 1], vst[HW][NQ / 2 > 0 ? NQ / 2 : 1];
  if constexpr (TR && DT::X32) {
    // Wave-private 1 KB blocks per (head, tensor, 32-feature part), key n's
    // row at 64 n: lane (g, n) writes features 4g + r and 16 + 4g + r and
    // reads back 8g .. 8g + 7. The last chunk's barrier has freed the LDS.
    static_assert(HP * NQ * 1024 <= Cfg::LDS_BYTES, "regather blocks exceed the LDS plan");
#pragma unroll
    for (int hl = 0; hl < HW; ++hl)
#pragma unroll
      for (int t = 0; t < NQ / 2; ++t) {
        unsigned char* bk = smem + (((w * HW + hl) * 2 + 0) * (NQ / 2) + t) * 1024 + n * 64;
        unsigned char* bv = smem + (((w * HW + hl) * 2 + 1) * (NQ / 2) + t) * 1024 + n * 64;
        *reinterpret_cast<bf16x4*>(bk + 8 * g) = pack4(dK[hl][2 * t]);
        *reinterpret_cast<bf16x4*>(bk + 32 + 8 * g) = pack4(dK[hl][2 * t + 1]);
        *reinterpret_cast<bf16x4*>(bv + 8 * g) = pack4(dV[hl][2 * t]);
        *reinterpret_cast<bf16x4*>(bv + 32 + 8 * g) = pack4(dV[hl][2 * t + 1]);
      }
    wave_lds_sync();
#pragma unroll
    for (int hl = 0; hl < HW; ++hl)
#pragma unroll
      for (int t = 0; t < NQ / 2; ++t) {
        kst[hl][t] = *reinterpret_cast<const bf16x8*>(smem + (((w * HW + hl) * 2 + 0) * (NQ / 2) + t) * 1024 + n * 64 + 16 * g);
        vst[hl][t] = *reinterpret_cast<const bf16x8*>(smem + (((w * HW + hl) * 2 + 1) * (NQ / 2) + t) * 1024 + n * 64 + 16 * g);
      }
  }
  if (key_ok) {
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
      const int h = w * HW + hl;
      if (h >= H) continue;
      bf16* krow = dkg + rx.off(h, my_key, D);
      bf16* vrow = dvg + rx.off(h, my_key, D);
      if constexpr (DT::X32) {
#pragma unroll
        for (int t = 0; t < NQ / 2; ++t) {
          if constexpr (TR) {
            *reinterpret_cast<bf16x8*>(krow + DT::dmap(2 * t, g, 0)) = kst[hl][t];
            *reinterpret_cast<bf16x8*>(vrow + DT::dmap(2 * t, g, 0)) = vst[hl][t];
          } else {
            *reinterpret_cast<bf16x8*>(krow + DT::dmap(2 * t, g, 0)) = cat8(pack4(dK[hl][2 * t]), pack4(dK[hl][2 * t + 1]));
            *reinterpret_cast<bf16x8*>(vrow + DT::dmap(2 * t, g, 0)) = cat8(pack4(dV[hl][2 * t]), pack4(dV[hl][2 * t + 1]));
          }
        }
      } else {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          *reinterpret_cast<bf16x4*>(krow + DT::dmap(q, g, 0)) = pack4(dK[hl][q]);
          *reinterpret_cast<bf16x4*>(vrow + DT::dmap(q, g, 0)) = pack4(dV[hl][q]);
        }
      }
    }
  }
  zero_tile_rows<bf16, D>(ev, rx, rx, k0, len, H, tid, dkg, nullptr);
  zero_tile_rows<bf16, D>(ev, rx, rx, k0, len, H, tid, dvg, nullptr);
}

// ---------------------------------------------------------------------------
// Dispatch.
// ---------------------------------------------------------------------------
template <int HP, int D, int C>
struct Bwd2Pick {
  static constexpr int KC = FST_ROWS_KC;  // keys per rows-kernel chunk
  static constexpr int HB = FST_ROWS_HB;  // heads per phase batch of the rows kernel
  static constexpr int RC = 16;  // rows per cols-kernel chunk
  // Waves of the rows kernel: eight where a four-wave lane's state would not
  // fit its registers. (HP / 4) D + 3 C tracks that state (the head-owner's
  // fragments and accumulators, the row-owner's H, G, u, w~); compiled for
  // gfx950, the four-wave instances spill from about 160 on and the
  // eight-wave ones fit (spills remain only at HP = 16 with D, C >= 48).
  static constexpr int NW = (HP % 8 == 0 && rows_wave_load(HP, D, C) >= 160) ? 8 : 4;
  static constexpr bool OK = Rows2Cfg<HP, D, C, KC, NW>::FITS && Cols2Cfg<HP, D, C, RC>::FITS;
  // Variants a caller may choose instead (the FST_PLAN_ROWS_* and
  // FST_PLAN_COLS_* bits); each computes every row with the same arithmetic.
  // The rows kernel at HP heads offers four waves below the spilling load,
  // eight in one workgroup per CU where HP is a multiple of 8 (the library
  // pads heads to 8 for that plan), eight in two workgroups per CU (four
  // waves per SIMD, a 128-register lane budget) below the spilling load, and
  // with either layout below the load its K and V rows staged in LDS where D
  // is a multiple of 32; the cols kernel offers three workgroups per CU
  // where its LDS plan fits a third of the CU and the lane state is that of
  // the small layouts ((HP / 4) D + 3 C < 160).
  static constexpr bool LIGHT = rows_wave_load(HP, D, C) < 160;
  static constexpr bool ROWS_W4 = Rows2Cfg<HP, D, C, KC, 4>::FITS && LIGHT;
  static constexpr bool ROWS_W8 = HP % 8 == 0 && Rows2Cfg<HP, D, C, KC, 8>::FITS;
  static constexpr bool ROWS_W8X2 = Rows2Cfg<HP, D, C, KC, 8, 4>::FITS && LIGHT;
  static constexpr bool KL_W4 = ROWS_W4 && Rows2Cfg<HP, D, C, KC, 4, 2, true>::FITS;
  static constexpr bool KL_W8X2 = ROWS_W8X2 && Rows2Cfg<HP, D, C, KC, 8, 4, true>::FITS;
  using CC = Cols2Cfg<HP, D, C, RC>;
  static constexpr bool COLS_OCC3 = CC::FITS && CC::LDS_BYTES <= 160 * 1024 / 3 && LIGHT;
  static constexpr int COLS_PLANS = CC::FITS ? (FST_PLAN_COLS_OCC2 | (COLS_OCC3 ? FST_PLAN_COLS_OCC3 : 0)) : 0;
  // Static choices among them, as measured on gfx950 with lengths U{16..L}:
  // where HP is a multiple of 8 and the lane state is light, eight rows-kernel
  // waves in two workgroups per CU (H=8, D=32, C=16: 0.567 against 0.636 ms
  // with four; H=16, D=C=16: 0.710 against 0.847), elsewhere four (H=12
  // gains nothing: its eight-wave split is uneven); the cols kernel at three
  // workgroups per CU wherever that is offered (H=8, D=48, C=16: 0.367
  // against 0.437 ms; within 1 % elsewhere).
  static constexpr int ROWS_STATIC = NW == 8 ? 2 : ((HP % 8 == 0 && ROWS_W8X2) ? 3 : 1);
  static constexpr int COLS_STATIC = COLS_OCC3 ? 3 : 2;
};

template <int HP, int D, int C, int NW, int WPE, bool KL>
int bwd2_launch_rows(const BwdParams& prm, hipStream_t stream, int g8, bool query) {
  using P = Bwd2Pick<HP, D, C>;
  using Cfg = Rows2Cfg<HP, D, C, P::KC, NW, WPE, KL>;
  if constexpr (!Cfg::FITS) {
    return FST_EUNSUPPORTED;
  } else {
    if (query) return FST_OK;
    // With the forward's output the rows kernel forms dS against a reference
    // D from it and corrects once at the end; without, D is formed online.
    const bool fb = (prm.flags & 3) == 3;
    auto kern = prm.out ? (fb ? bwd_rows2_kernel<HP, D, C, P::KC, P::HB, 3, NW, WPE, KL, true>
                              : bwd_rows2_kernel<HP, D, C, P::KC, P::HB, -1, NW, WPE, KL, true>)
                        : (fb ? bwd_rows2_kernel<HP, D, C, P::KC, P::HB, 3, NW, WPE, KL, false>
                              : bwd_rows2_kernel<HP, D, C, P::KC, P::HB, -1, NW, WPE, KL, false>);
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::LDS_BYTES) !=
        hipSuccess)
      return FST_ELAUNCH;
    if (g8 > 0) hipLaunchKernelGGL(kern, dim3(g8), dim3(64 * NW), Cfg::LDS_BYTES, stream, prm);
    return hipGetLastError() == hipSuccess ? FST_OK : FST_ELAUNCH;
  }
}

template <int HP, int D, int C, int OCC>
int bwd2_launch_cols(const BwdParams& prm, hipStream_t stream, int g8, bool query) {
  using P = Bwd2Pick<HP, D, C>;
  using Cfg = Cols2Cfg<HP, D, C, P::RC>;
  if (query) return FST_OK;
  // One instance per bias-flag combination: a kernel reading the flags at
  // run time keeps both bias paths live and spills at the larger layouts.
  const int fl = prm.flags & 3;
  auto kern = fl == 3   ? bwd_cols2_kernel<HP, D, C, P::RC, 3, OCC>
              : fl == 1 ? bwd_cols2_kernel<HP, D, C, P::RC, 1, OCC>
              : fl == 2 ? bwd_cols2_kernel<HP, D, C, P::RC, 2, OCC>
                        : bwd_cols2_kernel<HP, D, C, P::RC, 0, OCC>;
  if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::LDS_BYTES) !=
      hipSuccess)
    return FST_ELAUNCH;
  if (g8 > 0) hipLaunchKernelGGL(kern, dim3(g8), dim3(256), Cfg::LDS_BYTES, stream, prm);
  return hipGetLastError() == hipSuccess ? FST_OK : FST_ELAUNCH;
}

// Launches (or, with query, only checks) the rows (which = 0) or cols
// (which = 1) kernel variant the plan bits of prm.flags name. For the rows
// kernel HP is the rows head padding, which the library rounds to a
// multiple of 8 when the eight-wave, one-workgroup plan (static or chosen)
// runs. FST_BWD_PART: the kernels a translation unit instantiates (0 both,
// 1 the rows kernel, 2 the cols kernel), so the rows kernel can be built
// with its own scheduler options; the launcher has internal linkage, as
// its body depends on the part.
#ifndef FST_BWD_PART
#define FST_BWD_PART 0
#endif
template <int HP, int D, int C>
static int bwd2_launch_t(const BwdParams& prm, int which, hipStream_t stream, int grid, bool query) {
  using P = Bwd2Pick<HP, D, C>;
  // The grid is rounded up to a multiple of 64 for the XCD schedules
  // (tile_block); logical blocks past the work list exit at once.
  const int g8 = grid > 0 ? (grid + 63) & ~63 : 0;
  const int f = prm.flags;
  if (which == 0) {
#if FST_BWD_PART == 2
    return FST_EUNSUPPORTED;
#else
    const bool kl = f & FST_PLAN_ROWS_KV_LDS;
    const int waves = (f & FST_PLAN_ROWS_W4)     ? 1
                      : (f & FST_PLAN_ROWS_W8)   ? 2
                      : (f & FST_PLAN_ROWS_W8X2) ? 3
                                                 : P::ROWS_STATIC;
    if (waves == 1) {
      if constexpr (P::ROWS_W4) {
        if (!kl) return bwd2_launch_rows<HP, D, C, 4, 2, false>(prm, stream, g8, query);
        if constexpr (P::KL_W4) return bwd2_launch_rows<HP, D, C, 4, 2, true>(prm, stream, g8, query);
      }
      return FST_EUNSUPPORTED;
    }
    if (waves == 2) {
      if constexpr (P::ROWS_W8)
        if (!kl) return bwd2_launch_rows<HP, D, C, 8, 2, false>(prm, stream, g8, query);
      return FST_EUNSUPPORTED;
    }
    if constexpr (P::ROWS_W8X2) {
      if (!kl) return bwd2_launch_rows<HP, D, C, 8, 4, false>(prm, stream, g8, query);
      if constexpr (P::KL_W8X2) return bwd2_launch_rows<HP, D, C, 8, 4, true>(prm, stream, g8, query);
    }
    return FST_EUNSUPPORTED;
#endif
  }
#if FST_BWD_PART == 1
  return FST_EUNSUPPORTED;
#else
  if constexpr (!P::CC::FITS) {
    return FST_EUNSUPPORTED;
  } else {
    const int occ = (f & FST_PLAN_COLS_OCC2) ? 2 : (f & FST_PLAN_COLS_OCC3) ? 3 : P::COLS_STATIC;
    if (occ == 3) {
      if constexpr (P::COLS_OCC3) return bwd2_launch_cols<HP, D, C, 3>(prm, stream, g8, query);
      return FST_EUNSUPPORTED;
    }
    return bwd2_launch_cols<HP, D, C, 2>(prm, stream, g8, query);
  }
#endif
}

}  // namespace fst
