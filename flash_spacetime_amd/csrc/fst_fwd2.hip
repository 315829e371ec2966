// Forward kernel of flash-spacetime attention for gfx950, bf16 operands.
//
// Spec: reference.py:106-167; fused algebra: forward.py:5-22. For every
// query row i, head h and key j of one event:
//   s_ij = qt_i . k_j + [A] u_i . E_ij         (u = bf16(qt @ W), qt = q*scale)
//   p_ij = softmax_j(s_ij)
//   out_i = sum_j p_ij v_j + [V] (W (sum_j p_ij E_ij) + b)
//
// One workgroup = one 16-row tile of one event, four waves. Wave w is
//  * head-owner of heads [w HW, (w+1) HW): S^T_h = K_h Qt_h^T + (u.E)^T and
//    O^T_h += V_h^T P^T_h on 16x16 MFMA tiles with the 16 rows on the lanes,
//    the online softmax and its row sums l (fp32, per lane group, summed
//    across the groups at the end);
//  * row-owner of rows 4w .. 4w+3: u of its rows (bf16 MFMA over W in two
//    parts), the embedding E of its rows x the chunk's keys, computed in the
//    operand layout of the u.E product (UE^T_i = E_i U_i^T, heads on the
//    lanes) and kept in LDS for A^T_i += E_i^T P_i^T (A = sum_j p_ij E_ij).
// The roles meet in LDS: u.E goes row-owner -> head-owner (fp32), P and the
// rescale factors head-owner -> row-owner; E is private to the wave that
// computed it. Two barriers per key chunk, LDS-only (lds_barrier): a
// workgroup fence there would also wait for the V rows' direct loads in
// flight.
//
// K comes from global memory in row-major operand layout. Where the LDS plan
// allows (D a multiple of 32), each chunk's V rows go straight to LDS by
// direct loads and are read transposed (QoTile); otherwise V^T is made on the
// matrix core (identity product). q, k and v are addressed through
// row_addr_x (token stride three times out's when they are the slots of one
// fused projection), out and lse through row_addr. Keys past the event are clamped to
// the last valid key for loads and masked to -inf in the last chunk only.
// The softmax reference m is raised only when a row's chunk maximum exceeds
// it by more than 2^8 (log2 domain), so O, l and A are rescaled rarely.
#include "fst_tile.h"

namespace fst {

template <int HP, int D, int C, int KC, int OCC>
struct Fwd2Cfg {
  static constexpr int HW = HP / 4;  // heads per wave
  static constexpr int NS = KC / 16;  // 16-key subtiles per chunk
  static constexpr int NCT = C / 16;  // channel steps
  static constexpr int E_BYTES = ETile<C, KC>::BYTES;
  static constexpr int STAGE_BYTES = (KC / 4) * 16 * 16 * 16;  // fp32 u.E of KC keys per (row, head)
  static constexpr int SCAL_BYTES = 16 * 17 * 4 + 16;  // rescale factors, then one flag per wave
  static constexpr int BASE_BYTES = E_BYTES + STAGE_BYTES + SCAL_BYTES;
  // VL: each chunk's V rows go straight to LDS (QoTile blocks, one per head
  // and 32-feature part) and are read transposed there, where D is a multiple
  // of 32, the chunk 16 keys and the blocks fit the occupancy's LDS share.
  static constexpr int V_BYTES = HP * (D / 32) * 1024;
  static constexpr bool VL = D % 32 == 0 && KC == 16 && BASE_BYTES + V_BYTES <= (160 / OCC) * 1024;
  static constexpr int LDS_BYTES = BASE_BYTES + (VL ? V_BYTES : 0);
  // OCC: workgroups per CU the register and LDS plan is built for.
  static constexpr bool FITS = LDS_BYTES <= (160 / OCC) * 1024 && HP % 4 == 0 && (KC == 16 || KC == 32);
};

constexpr float kRescaleLog2 = 8.f;

template <int HP, int D, int C, int KC, int OCC, int FL>
__global__ __launch_bounds__(256, OCC) void fwd2_kernel(FwdParams prm) {
  using Cfg = Fwd2Cfg<HP, D, C, KC, OCC>;
  using ET = ETile<C, KC>;
  using DT = DTiles<D>;
  constexpr int HW = Cfg::HW, NS = Cfg::NS, NCT = Cfg::NCT, NQ = DT::NQ;
  constexpr bool VL = Cfg::VL;
  constexpr int NP = D / 32;  // 32-feature parts of a row (VL)
  extern __shared__ __align__(16) unsigned char smem[];
  bf16* Es = reinterpret_cast<bf16*>(smem);
  unsigned char* stage = smem + Cfg::E_BYTES;
  unsigned char* scal = stage + Cfg::STAGE_BYTES;
  int* rflag = reinterpret_cast<int*>(scal + 16 * 17 * 4);  // wave w rescaled its heads this chunk
  unsigned char* vtile = smem + Cfg::BASE_BYTES;  // VL: [head][part] QoTile blocks of the chunk's V

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
  const RowAddr ra = row_addr(prm.ev, eb);   // out, lse
  const RowAddr rx = row_addr_x(prm.ev, eb);  // q, k, v
  const int i0 = eb.blk * 16;
  const int last = len - 1;
  bf16* outg = reinterpret_cast<bf16*>(prm.out);
  if (event_refused(prm.ev, eb)) {
    fill_rows_nan<bf16, D>(ra, ra, i0, min(i0 + 16, len), H, tid, 256, outg, prm.lse);
    return;
  }
  if (i0 >= len) {  // a tile of padding rows only
    zero_tile_rows<bf16, D>(prm.ev, ra, ra, i0, len, H, tid, outg, prm.lse);
    return;
  }

  const bf16* __restrict__ qg = reinterpret_cast<const bf16*>(prm.q);
  const bf16* __restrict__ kg = reinterpret_cast<const bf16*>(prm.k);
  const bf16* __restrict__ vg = reinterpret_cast<const bf16*>(prm.v);
  const bf16x4 id = ident_x16(g, n);

  // ---- head-owner state (lane n = row i0 + n) ----
  const int my_row = i0 + n;
  const bool row_ok = my_row < len;
  KFrag<bf16, D> qf[HW];
  f32x4 O[HW][NQ];
  float lsum[HW];  // this lane group's part of the row sum
  float mref[HW];
  // The prologue's loads (q, W, the projected rows, positions, then the
  // first chunk's operands) are all issued before the first of them is used,
  // from clamped rows and without branches, so none waits for another.
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    // Padded heads (h >= H) compute on head H-1's data and are never stored,
    // so the chunk loop needs no per-head branches.
    const int hq = min(w * HW + hl, H - 1);
    qf[hl].load(qg + rx.off(hq, row_ok ? my_row : last, D), g);
  }

  // ---- row-owner state: rows i0 + 4w + r, heads on lane n ----
  WSlots<D, C> wv;
  SlotRow<D> xq[4];
  if (attn) {
    wv.load(prm.weight, g, n);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = i0 + 4 * w + r;
      xq[r].load(qg + rx.off(0, row < len ? row : last, D), rx.hs * D, row < len && n < H, g, n);
    }
  }
  // Angle lane assignment: lane (g, n) evaluates row i0 + 4w + g against key
  // j0 + 16 s + n; the four rows are then gathered into every lane group.
  float4 pos_i = float4{0.f, 0.f, 0.f, 0.f};
  float fa[NCT], fb[NCT];
  if (use_e) {
    const int row = i0 + 4 * w + g;
    pos_i = ra.pos(prm.ev.pos4, row < len ? row : last);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      fa[ct] = 1024.f * prm.freq.ghi[8 * ct + 2 * g];
      fb[ct] = 1024.f * prm.freq.ghi[8 * ct + 2 * g + 1];
    }
  }

  // Buffer views of this event's K, V and positions. Row r of head h sits at
  // element (r ts + h hs) D from the event's base; a chunk advances the
  // scalar offset by KC ts D elements.
  const long ebase = rx.off(0, 0, D);
  const int rowb = (int)(rx.ts * D * 2);  // bytes per key row
  const unsigned ebytes = (unsigned)((prm.ev.tokmajor ? (long)len * rx.ts : (long)H * rx.hs) * D * 2);
  const Buf kbuf(kg + ebase, ebytes), vbuf(vg + ebase, ebytes);
  const Buf pbuf(prm.ev.pos4 + ra.pos_base, (unsigned)len * 16u);
  int kvo[HW];  // lane offset of head hl, key n (bytes)
#pragma unroll
  for (int hl = 0; hl < HW; ++hl)
    kvo[hl] = (int)(min(w * HW + hl, H - 1) * rx.hs * D * 2) + n * rowb + kfrag_goff<D>(g);

  // Operands of the chunk in flight: K, V rows of the wave's heads and the
  // key positions. Loads for chunk j0 + KC are issued as soon as the
  // head-owner has consumed those of chunk j0; keys are clamped to the event.
  // Every chunk issues the same loads in the same order (positions, then K
  // and V; past the last chunk they reread clamped keys), so the wait at the
  // top of a chunk covers the positions only and E is formed while K and V
  // are still in flight.
  KFrag<bf16, D> kf[HW][NS], vf[VL ? 1 : HW][NS];
  float4 pj[NS];
  // NF: chunk jn is known to be whole (no clamped keys), so its addresses
  // need no selects.
  auto issue = [&](int jn, auto nf_tag) __attribute__((always_inline)) {
    const bool full = decltype(nf_tag)::value || jn + KC <= len;
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int voff = full ? kvo[hl] + 16 * s * rowb : kvo[hl] + (min(jn + 16 * s + n, last) - n) * rowb;
        const int soff = full ? jn * rowb : 0;
        load_kfrag<D>(kf[hl][s], kbuf, voff, soff);
        if constexpr (!VL) load_kfrag<D>(vf[hl][s], vbuf, voff, soff);
      }
    }
  };
  // VL: the wave's heads' V rows of chunk jn straight to LDS, lane l of a
  // block load fetching the quarter QoTile keeps in slot l; keys past the
  // event are clamped to its last key (their P is zero).
  const int vo_r = lane >> 2, vo_c = (lane & 3) ^ QoTile::swz(vo_r);
  auto issue_v = [&](int jn) __attribute__((always_inline)) {
    if constexpr (VL) {
      const bool full = jn + KC <= len;
      const int rel = full ? vo_r * rowb : min(jn + vo_r, last) * rowb;
      const int soff = full ? jn * rowb : 0;
#pragma unroll
      for (int hl = 0; hl < HW; ++hl) {
        const int h = w * HW + hl;
        const int voff = (int)(min(h, H - 1) * rx.hs * D * 2) + rel + 16 * vo_c;
#pragma unroll
        for (int t = 0; t < NP; ++t)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(vbuf.r, (__attribute__((address_space(3))) void*)(vtile + (h * NP + t) * 1024),
                                                   16, voff + 64 * t, soff, 0, 0);
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
  issue_pos(0, std::false_type{});
  issue(0, std::false_type{});

#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    // Without a branch: the compiler would sink the q loads into it, each
    // then waited for with every load before it.
    qf[hl].scale_by(prm.scale);
    qf[hl].keep_if(row_ok);
#pragma unroll
    for (int q = 0; q < NQ; ++q) O[hl][q] = zero4();
    lsum[hl] = 0.f;
    mref[hl] = -INFINITY;
  }
  bf16x4 uf[4][NCT];
  f32x4 AE[4][NCT];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (attn) {
      // u^T[slot][h] = scale sum_d W[d][channel(slot)] q[h][d] (project_loaded).
      project_loaded<D, C>(xq[r], i0 + 4 * w + r < len && n < H, prm.scale, wv, uf[r]);
    } else {
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) uf[r][ct] = bf16x4{};
    }
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) AE[r][ct] = zero4();
  }

  // next_tag: the next chunk is whole (its prefetch addresses need no clamps).
  auto chunk = [&](int j0, auto tail_tag, auto next_tag) __attribute__((always_inline)) {
    constexpr bool TAIL = decltype(tail_tag)::value;
    issue_v(j0);  // lands during the row-owner part

    // ---- row-owner: E of rows 4w..4w+3 x KC keys; u.E staged ----
    if (use_e) {
      float xg[NS][4];
#pragma unroll
      for (int s = 0; s < NS; ++s) group_gather(pair_angle_unit(pos_i, pj[s]), xg[s]);
      // No prefetch past the last chunk (its loads would only hold the
      // epilogue back).
      if (decltype(next_tag)::value || j0 + KC < len) issue_pos(j0 + KC, next_tag);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          bf16x4 ef[NCT];
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) {
            ef[ct] = embed_step<C>(xg[s][r], fa[ct], fb[ct], ct);
            if (act) ET::store(Es, 4 * w + r, ct, 16 * s + n, g, ef[ct]);
          }
          if (attn) {
            f32x4 ue = zero4();
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) ue = mfma_x16(ef[ct], uf[r][ct], ue);
            *reinterpret_cast<f32x4*>(stage + stage_off(4 * s + g, 4 * w + r, n)) = ue;
          }
          // One (row, subtile) at a time: the scheduler's own interleaving of
          // the rows measured 2 % slower.
          __builtin_amdgcn_sched_barrier(0);
        }
    }
    lds_barrier();  // u.E staged
    // Wave priority by phase: the row-owner phase (its MFMAs feed the next
    // chunk's u.E) runs at 1, the head-owner phase at 0 (-2 % forward).
    __builtin_amdgcn_s_setprio(0);

    // ---- head-owner: logits, online softmax, P V (phase by phase over the
    // wave's heads, so the heads' dependency chains overlap) ----
    f32x4 S[HW][NS];
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const f32x4 init =
            attn ? *reinterpret_cast<const f32x4*>(stage + stage_off(4 * s + g, n, w * HW + hl)) : zero4();
        S[hl][s] = mma_k<D>(kf[hl][s], qf[hl], init);
        if constexpr (TAIL) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (j0 + 16 * s + 4 * g + r >= len) S[hl][s][r] = -INFINITY;
        }
      }
    }
    // A row's reference m moves only when some key of the chunk exceeds it by
    // more than 2^8. X holds the exponents of the chunk's probabilities against
    // the current reference; each lane tests the largest of its own, and only
    // then is the row maximum formed across the lane groups. (On the first
    // chunk the reference is -inf and every valid key's X is +inf.)
    float mx[HW], alpha[HW];
    f32x4 X[HW][NS];
    float margin = -INFINITY;
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
      const float mb = mref[hl];
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          X[hl][s][r] = __builtin_fmaf(S[hl][s][r], kLog2e, -mb);
          margin = fmaxf(margin, X[hl][s][r]);
        }
      alpha[hl] = 1.f;
    }
    const bool rescale = __builtin_amdgcn_ballot_w64(margin > kRescaleLog2) != 0;
    if (rescale) {
#pragma unroll
      for (int hl = 0; hl < HW; ++hl) {
        float m = S[hl][0][0];
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) m = fmaxf(m, S[hl][s][r]);
        mx[hl] = group_allmax(m * kLog2e);
        const float mnew = mx[hl] > mref[hl] + kRescaleLog2 ? mx[hl] : mref[hl];
        alpha[hl] = exp2f_fast(mref[hl] - mnew);
        mref[hl] = mnew;
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) X[hl][s][r] = __builtin_fmaf(S[hl][s][r], kLog2e, -mnew);
#pragma unroll
        for (int q = 0; q < NQ; ++q) O[hl][q] = O[hl][q] * alpha[hl];
        lsum[hl] *= alpha[hl];
      }
    }
    JFrag<bf16, NS> pf[HW];
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
      float ls = lsum[hl];
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          S[hl][s][r] = exp2f_fast(X[hl][s][r]);
          ls += S[hl][s][r];
        }
      lsum[hl] = ls;
      pf[hl].from_tiles(S[hl]);
    }
    // This wave's V rows are in LDS (VL): only its own loads need waiting
    // for, and the previous chunk's reads of the blocks ended at its closing
    // barrier.
    if constexpr (VL) wait_vmem();
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        JFrag<bf16, NS> vt;
        if constexpr (VL)
          vt.v = QoTile::tr_frag_dmap(vtile + ((w * HW + hl) * NP + (q >> 1)) * 1024, q, g, n);
        else if constexpr (NS == 2)
          vt.v = cat8(transpose_x16(DT::part(vf[hl][0], q), id), transpose_x16(DT::part(vf[hl][1], q), id));
        else
          vt.v = transpose_x16(DT::part(vf[hl][0], q), id);
        O[hl][q] = mma_j(vt, pf[hl], O[hl][q]);
      }
    }
    if (act) {
      // P for the row-owner: keys 16s + 4g .. +3 of slot (row n, head h).
#pragma unroll
      for (int hl = 0; hl < HW; ++hl) {
        const int h = w * HW + hl;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          bf16x4 pv;
#pragma unroll
          for (int r = 0; r < 4; ++r) pv[r] = pf[hl].v[4 * s + r];
          *reinterpret_cast<bf16x4*>(stage + half_off(2 * s + (g >> 1), n, h, g & 1)) = pv;
        }
        // Only a wave that rescaled writes its factors (the same value from
        // every lane group); its flag tells the row-owners to read them.
        if (rescale) *reinterpret_cast<float*>(scal + scal_off(n, h)) = alpha[hl];
      }
      rflag[w] = rescale ? 1 : 0;
    }
    if (decltype(next_tag)::value || j0 + KC < len) issue(j0 + KC, next_tag);
    __builtin_amdgcn_s_setprio(1);
    lds_barrier();  // P and rescale factors staged

    // ---- row-owner: A = alpha A + E^T P ----
    if (act) {
      const int4 fl = *reinterpret_cast<const int4*>(rflag);
      if (__builtin_amdgcn_readfirstlane(fl.x | fl.y | fl.z | fl.w)) {
        // Rare: some head-owner moved its reference m this chunk. (The empty
        // volatile asm keeps this a branch rather than selects.)
        __asm__ volatile("");
        const int ow = n / HW;  // the wave that owns head n
        const bool fresh = n < H && (ow == 0 ? fl.x : ow == 1 ? fl.y : ow == 2 ? fl.z : fl.w) != 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float al = *reinterpret_cast<const float*>(scal + scal_off(4 * w + r, n));
          const float alpha = fresh ? al : 1.f;
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) AE[r][ct] = AE[r][ct] * alpha;
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int il = 4 * w + r;
        JFrag<bf16, NS> pr;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const bf16x4 pv =
              *reinterpret_cast<const bf16x4*>(stage + half_off(2 * s + (g >> 1), il, n, g & 1));
#pragma unroll
          for (int e = 0; e < 4; ++e) pr.v[4 * s + e] = pv[e];
        }
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
          JFrag<bf16, NS> et;
          if constexpr (NS == 2)
            et.v = cat8(ET::load_tr(Es, il, ct, 0, g, n), ET::load_tr(Es, il, ct, 16, g, n));
          else
            et.v = ET::load_tr(Es, il, ct, 0, g, n);
          AE[r][ct] = mma_j(et, pr, AE[r][ct]);
        }
      }
    }
  };

  int j0 = 0;
  for (; j0 + 2 * KC <= len; j0 += KC) chunk(j0, std::false_type{}, std::true_type{});
  if (j0 + KC <= len) {
    chunk(j0, std::false_type{}, std::false_type{});
    j0 += KC;
  }
  if (j0 < len) chunk(j0, std::true_type{}, std::false_type{});

  // ---- epilogue ----
  // O's accumulator q holds features omap(q, g, r) = DTiles::dmap(q, g, r)
  // (V read transposed from LDS in that order where VL): four consecutive
  // features, eight across the pair 2t, 2t + 1 where D is a multiple of 32.
  auto omap = [&](int q, int gg, int r) { return DT::dmap(q, gg, r); };
  // The epilogue's operands are loaded first, ahead of the lse stores (the
  // compiler would issue them only after those, on the epilogue's chain):
  // b, by buffer loads whose range is empty, reading zeros, when there is no
  // b, and W as two bf16 parts per head-dim tile (lane n of the W operand is
  // the tile's feature omap(q, n/4, n%4)) where those take few registers
  // (NQ NCT <= 2; otherwise each round loads its own).
  constexpr bool WPRE = NQ * NCT <= 2;
  bf16x4 wh[NQ][NCT], wl[NQ][NCT];
  f32x4 bq[NQ];
  auto load_w = [&](int q) __attribute__((always_inline)) {
    const int dn = omap(q, n >> 2, n & 3);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      f32x4 wq;
#pragma unroll
      for (int sp = 0; sp < 4; ++sp) wq[sp] = prm.weight[dn * C + slot_channel<C>(16 * ct + 4 * g + sp)];
      split4(wq, wh[q][ct], wl[q][ct]);
    }
  };
  if (act) {
    const Buf bb(prm.bias, prm.bias ? D * 4 : 0);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if constexpr (WPRE) load_w(q);
      const float4 b4 = bb.ldf4(omap(q, g, 0) * 4, 0);
      bq[q] = f32x4{b4.x, b4.y, b4.z, b4.w};
    }
  }
  float inv_l[HW];
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    const float l = group_allsum(lsum[hl]);
    inv_l[hl] = 1.f / l;
    const int h = w * HW + hl;
    if (g == 0 && row_ok && h < H) prm.lse[ra.vec(h, my_row)] = mref[hl] * kLn2 + __logf(l);
  }

  // One head-dim tile per round: the row-owner forms o2^T_i[d, h] =
  // sum_slot W[d, channel(slot)] A^T_i[slot, h] on bf16 MFMA over the two
  // parts of each factor (W and A to 16 bits) and stages it; the head-owner
  // forms out = (O + o2) / l + b in place.
  bf16x4 aeh[4][NCT], ael[4][NCT];
  if (act) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) split4(AE[r][ct], aeh[r][ct], ael[r][ct]);
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    if (act) {
      if constexpr (!WPRE) load_w(q);
      __syncthreads();  // previous round (or the last chunk) done with the stage
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        f32x4 acc = zero4();
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) acc = mma_split(wh[q][ct], wl[q][ct], aeh[r][ct], ael[r][ct], acc);
        *reinterpret_cast<f32x4*>(stage + stage_off(g, 4 * w + r, n)) = acc;
      }
      __syncthreads();
    }
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
      f32x4 o = O[hl][q];
      if (act) o = o + *reinterpret_cast<const f32x4*>(stage + stage_off(g, n, w * HW + hl));
      o = o * inv_l[hl];
      if (act) o = o + bq[q];
      O[hl][q] = o;
    }
  }
  if (row_ok) {
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
      const int h = w * HW + hl;
      if (h >= H) continue;
      bf16* orow = outg + ra.off(h, my_row, D);
      if constexpr (DT::X32) {
#pragma unroll
        for (int t = 0; t < NQ / 2; ++t)
          *reinterpret_cast<bf16x8*>(orow + DT::dmap(2 * t, g, 0)) = cat8(pack4(O[hl][2 * t]), pack4(O[hl][2 * t + 1]));
      } else {
#pragma unroll
        for (int q = 0; q < NQ; ++q) *reinterpret_cast<bf16x4*>(orow + DT::dmap(q, g, 0)) = pack4(O[hl][q]);
      }
    }
  }

  zero_tile_rows<bf16, D>(prm.ev, ra, ra, i0, len, H, tid, outg, prm.lse);
}

template <int HP, int D, int C>
struct Fwd2Pick {
  static constexpr int KC = 16;  // the static choice's keys per chunk
  // Three workgroups per CU where the LDS plan fits a third of the CU and the
  // lane state stays near the 168 registers of that budget ((HP / 4) D + 3 C
  // < 160: beyond it the instances spill); two otherwise. Measured on the
  // small layouts, the extra waves hide more latency than the smaller LDS
  // share costs (16-key chunks at three beat 32-key chunks at two), and at
  // the other layouts three is as fast or faster (HP = 16, D = C = 16: -23 %;
  // HP = 12, D = 16, C = 32: -19 %).
  static constexpr bool OCC3 = Fwd2Cfg<HP, D, C, KC, 3>::FITS && rows_wave_load(HP, D, C) < 160;
  static constexpr bool OCC2 = Fwd2Cfg<HP, D, C, KC, 2>::FITS;
  static constexpr int OCC = OCC3 ? 3 : 2;
  using Cfg = Fwd2Cfg<HP, D, C, KC, OCC>;
  static constexpr bool OK = Cfg::FITS;
  // 32-key chunks (FST_PLAN_FWD_KC32) at two workgroups per CU, where their
  // LDS plan fits and the lane state is that of the small layouts.
  static constexpr bool KC32 = OK && Fwd2Cfg<HP, D, C, 32, 2>::FITS && rows_wave_load(HP, D, C) < 160;
  // Occupancy and key-chunk variants a caller may choose instead (the plan
  // bits of include/flash_spacetime.h); the occupancy variants compute every
  // row with the same arithmetic.
  static constexpr int PLANS = OK ? ((OCC2 ? FST_PLAN_FWD_OCC2 : 0) | (OCC3 ? FST_PLAN_FWD_OCC3 : 0) |
                                     FST_PLAN_FWD_KC16 | (KC32 ? FST_PLAN_FWD_KC32 : 0))
                                  : 0;
};

template <int HP, int D, int C, int KC, int OCC>
int fwd2_launch_occ(const FwdParams& prm, hipStream_t stream, int grid, bool query) {
  using Cfg = Fwd2Cfg<HP, D, C, KC, OCC>;
  using P = Fwd2Pick<HP, D, C>;
  constexpr bool OFFERED = KC == 16 ? (OCC == 2 ? P::OCC2 : P::OCC3) : (P::KC32 && OCC == 2);
  if constexpr (!Cfg::FITS || !OFFERED) {
    return FST_EUNSUPPORTED;
  } else {
    if (query) return FST_OK;
    // Both bias flags (the operators' default) run an instance with the flags
    // fixed at compile time; other combinations read them at run time.
    auto kern = (prm.flags & 3) == 3 ? fwd2_kernel<HP, D, C, KC, OCC, 3> : fwd2_kernel<HP, D, C, KC, OCC, -1>;
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::LDS_BYTES) !=
        hipSuccess)
      return FST_ELAUNCH;
    // The grid is rounded up to a multiple of 64 for the XCD schedules
    // (tile_block); logical blocks past the work list exit at once.
    const int g8 = (grid + 63) & ~63;
    if (grid > 0) hipLaunchKernelGGL(kern, dim3(g8), dim3(256), Cfg::LDS_BYTES, stream, prm);
    return hipGetLastError() == hipSuccess ? FST_OK : FST_ELAUNCH;
  }
}

// Launches (or, with query, only checks) the variant the plan bits of
// prm.flags name: an empty occupancy group takes the static occupancy (two
// with 32-key chunks), an empty key-chunk group 16 keys.
template <int HP, int D, int C>
int fwd2_launch_t(const FwdParams& prm, hipStream_t stream, int grid, bool query) {
  using P = Fwd2Pick<HP, D, C>;
  if constexpr (!P::OK) {
    return FST_EUNSUPPORTED;
  } else {
    const bool kc32 = prm.flags & FST_PLAN_FWD_KC32;
    const int occ = (prm.flags & FST_PLAN_FWD_OCC2) ? 2 : (prm.flags & FST_PLAN_FWD_OCC3) ? 3 : (kc32 ? 2 : P::OCC);
    if (kc32) return occ == 2 ? fwd2_launch_occ<HP, D, C, 32, 2>(prm, stream, grid, query) : FST_EUNSUPPORTED;
    if (occ == 3) return fwd2_launch_occ<HP, D, C, 16, 3>(prm, stream, grid, query);
    return fwd2_launch_occ<HP, D, C, 16, 2>(prm, stream, grid, query);
  }
}

}  // namespace fst
