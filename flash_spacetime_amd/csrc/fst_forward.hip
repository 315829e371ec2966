// Fused forward kernel of flash-spacetime attention for gfx950.
//
// Spec: reference.py:106-167; fused algebra: forward.py:5-22. For every
// query row i, head h and key j of one event:
//   s_ij = qt_i . k_j + [A] u_i . E_ij         (u = T(qt @ W), qt = q*scale)
//   p_ij = softmax_j(s_ij)
//   out_i = sum_j p_ij v_j + [V] (W (sum_j p_ij E_ij) + b)
// The row-constant qt_i . b term of the logits is dropped (softmax shift),
// sum_j p_ij = 1 folds b out of the value sum, and E (C sin/cos channels of
// the pair's interval angle) is recomputed per tile and never stored.
//
// Work decomposition. A workgroup of WPG waves (four, or eight where NW is
// eight) owns ROWS query rows of one event, split in 16-row tiles; each tile
// is served by NW waves (NW in {1, 2, 4, 8}) that split the work two ways:
//  * head-owner role: wave ws of the tile owns heads [ws*HW, (ws+1)*HW) for
//    all 16 rows -- the per-head products S^T_h = K_h Qt_h^T and
//    O^T_h += V_h^T P^T_h on 16x16 MFMA tiles with rows on the lanes, and
//    the online softmax;
//  * row-owner role: wave ws owns rows [ws*RW, (ws+1)*RW) of the tile for
//    all heads -- u = qt W, the pair embedding E, and the per-row products
//    UE^T_i = E_i U_i (keys x heads) and AE^T_i += E_i^T P_i (channels x
//    heads), which carry the head index on the lanes.
// The two layouts meet in LDS: the row-owner stages u.E for the head-owner
// (fp32), the head-owner stages P and the rescale factors for the
// row-owner. A (row, head) staging slot is read (u.E) and then written (P)
// by the same head-owner wave, so the two share storage. Keys are processed
// in chunks of KC = 16*NS. For bf16, V is staged once per chunk for the whole
// workgroup and read with transposing LDS loads; fp32 reads V from global
// memory. K is read straight from global memory (it is already in
// MFMA-operand order) and the embedding stays in LDS for both consumers.
#include "fst_kernels.h"

namespace fst {

template <typename T, int HP, int D, int C, int NW, int NS>
struct FwdCfg {
  static constexpr bool BF = is_bf16<T>::value;
  static constexpr int HW = HP / NW;     // heads per head-owner wave
  static constexpr int RW = 16 / NW;     // rows per row-owner wave
  static constexpr int WPG = NW > 4 ? NW : 4;  // waves per workgroup
  static constexpr int THREADS = 64 * WPG;
  static constexpr int TILES = WPG / NW;  // 16-row tiles per workgroup
  static constexpr int ROWS = 16 * TILES;
  static constexpr int KC = 16 * NS;     // keys per chunk
  static constexpr int ESZ = sizeof(T);
  static constexpr int PAD = 16 / ESZ;   // 16 bytes of padding per LDS row
  // LDS regions. Row strides keep every vector access 16-byte aligned and
  // are padded to spread banks.
  static constexpr int V_ROW = D + PAD;                    // elements per key row of K and V
  static constexpr int E_ROW = C + PAD;                    // elements per (row, key)
  static constexpr int E_TILE = 16 * KC * E_ROW * ESZ;
  static constexpr int U_ROW = KC + 4;                     // fp32 u.E keys per slot
  static constexpr int P_ROW = KC + PAD;                   // T probabilities per slot
  static constexpr int O_ROW = 16 + 4;                     // fp32 o2 d-tile per slot
  static constexpr int SLOT_A = U_ROW * 4 > P_ROW * ESZ ? U_ROW * 4 : P_ROW * ESZ;
  static constexpr int SLOT = SLOT_A > O_ROW * 4 ? SLOT_A : O_ROW * 4;  // bytes per (row, head)
  static constexpr int STAGE_TILE = 16 * HP * SLOT;
  static constexpr int A_TILE = HP * 16 * 4;               // alpha[h][row]
  static constexpr int TILE_BYTES = E_TILE + STAGE_TILE + A_TILE;
  // Staging of each chunk's key rows in LDS by the whole workgroup
  // (coalesced 16-byte loads): V for bf16. KS (K as well) and float32 V are
  // kept off: for float32 the staged LDS plan halved the workgroups per CU
  // at B=256 L=768 H=12 D=32 C=16 (5.29 against 2.85 ms) and changed
  // nothing at cfg4, so float32 reads K fragments and gathers V transposed
  // from global memory.
  static constexpr int KV_ONE = HP * KC * V_ROW * ESZ;
  static constexpr bool VS = BF;
  static constexpr bool KS = false;
  static constexpr int V_BYTES = (VS ? KV_ONE : 0) + (KS ? KV_ONE : 0);  // V, then K
  static constexpr int LDS_BYTES = V_BYTES + TILES * TILE_BYTES;
  // VE (float32): each head's V columns are gathered before its logits
  // instead of right before P V, where the LDS plan already keeps one
  // workgroup per CU (over 80 KB): cfg4 forward 11.52 -> 11.10 ms; where the
  // registers cost a workgroup per CU it lost (B=256 L=768 H=12 D=32 C=16:
  // 2.87 -> 3.75 ms; H = 8, D = 32: 0.53 -> 0.60).
  static constexpr bool VE = !VS && LDS_BYTES > 80 * 1024;
  // A row-owner wave's RW rows x KC keys: whole embeddings per lane, or
  // whole groups of four frequencies per lane where lanes share a pair.
  using EL = EmbedLanes<RW * KC>;
  static constexpr bool FITS = LDS_BYTES <= 160 * 1024 && HP % NW == 0 && EL::OK && (C / 2 / EL::SPLIT) % 4 == 0 &&
                               !(BF && NS != 1 && NS != 2);
  static_assert(SLOT % 16 == 0, "slots must stay 16-byte aligned");
};

template <typename T, int HP, int D, int C, int NW, int NS>
__global__ __launch_bounds__(64 * (NW > 4 ? NW : 4), 1) void fwd_kernel(FwdParams prm) {
  using Cfg = FwdCfg<T, HP, D, C, NW, NS>;
  constexpr int NT = Cfg::THREADS;
  constexpr int HW = Cfg::HW, RW = Cfg::RW, KC = Cfg::KC;
  constexpr int SLOT_F = Cfg::SLOT / 4;          // slot stride in floats
  constexpr int SLOT_T = Cfg::SLOT / Cfg::ESZ;   // slot stride in T
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int tile = wave / NW, ws = wave % NW;

  // ---- work item: (event, row block) from the per-event block prefix ----
  EventBlock eb;
  if (!locate_block(prm.ev, blockIdx.x, eb)) return;
  const int len = eb.len;
  const int H = prm.H;
  const bool attn = prm.flags & FST_ATTN_BIAS;
  const bool act = prm.flags & FST_ACT_BIAS;
  const bool use_e = attn || act;
  const RowAddr ra = row_addr(prm.ev, eb);   // out, lse
  const RowAddr rx = row_addr_x(prm.ev, eb);  // q, k, v

  const int row0 = eb.blk * Cfg::ROWS;
  const int i0 = row0 + 16 * tile;  // first row of this wave's tile
  if (event_refused(prm.ev, eb)) {
    fill_rows_nan<T, D>(ra, ra, row0, min(row0 + Cfg::ROWS, len), H, tid, NT, reinterpret_cast<T*>(prm.out),
                        prm.lse);
    return;
  }

  T* Vs = reinterpret_cast<T*>(smem);
  T* Ks = Vs + HP * KC * Cfg::V_ROW;  // KS
  unsigned char* tbase = smem + Cfg::V_BYTES + tile * Cfg::TILE_BYTES;
  T* Es = reinterpret_cast<T*>(tbase);                                          // [16][KC][E_ROW]
  float* Sf = reinterpret_cast<float*>(tbase + Cfg::E_TILE);                    // [16][HP] slots
  T* St = reinterpret_cast<T*>(tbase + Cfg::E_TILE);                            // same slots as T
  float* As = reinterpret_cast<float*>(tbase + Cfg::E_TILE + Cfg::STAGE_TILE);  // [HP][16]

  const T* __restrict__ qg = reinterpret_cast<const T*>(prm.q);
  const T* __restrict__ kg = reinterpret_cast<const T*>(prm.k);
  const T* __restrict__ vg = reinterpret_cast<const T*>(prm.v);

  // ---- head-owner state: queries of its heads for the 16 rows (lane n) ----
  const int my_row = i0 + n;
  const bool row_ok = my_row < len;
  KFrag<T, D> qf[HW];
  f32x4 O[HW][D / 16];
  float m_run[HW], l_run[HW];
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    const int h = ws * HW + hl;
    if (h < H && row_ok)
      qf[hl].load_scaled(qg + rx.off(h, my_row, D), g, prm.scale);
    else
      qf[hl].zero();
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) O[hl][dt] = zero4();
    m_run[hl] = -INFINITY;
    l_run[hl] = 0.f;
  }

  // ---- row-owner state: u of its rows (lane n = head), AE accumulators ----
  CFrag<T, C> uf[RW];
  f32x4 AE[RW][C / 16];
#pragma unroll
  for (int ri = 0; ri < RW; ++ri) {
    const int row = i0 + ws * RW + ri;
    if (attn) {
      f32x4 acc[C / 16];
      const bool ok = row < len && n < H;
      project_row<T, D, C>(qg + rx.off(0, ok ? row : 0, D), rx.hs * D, ok, prm.scale, prm.weight, g, n, acc);
      uf[ri].from_acc(acc);
    } else {
      uf[ri].zero();
    }
#pragma unroll
    for (int ct = 0; ct < C / 16; ++ct) AE[ri][ct] = zero4();
  }
  // Pair-embedding assignment (EmbedLanes): lane slot el -> key (el % KC),
  // rows spaced by 64 / KC starting at el / KC.
  using EL = typename Cfg::EL;
  constexpr int EPL = EL::EPL;  // embeddings per lane per chunk
  constexpr int ESTEP = 64 / KC;
  const int el = EL::slot(lane), epart = EL::part(lane);
  float4 pos_i[EPL];
#pragma unroll
  for (int k2 = 0; k2 < EPL; ++k2) {
    const int row = i0 + ws * RW + el / KC + ESTEP * k2;
    pos_i[k2] = use_e ? ra.pos(prm.ev.pos4, row < len ? row : (len > 0 ? len - 1 : 0)) : float4{0.f, 0.f, 0.f, 0.f};
  }

  // PP: key positions run a chunk ahead, as the embedding needs them first
  // thing in a chunk (B=256 L=768 H=12 D=32 C=16 in float32: 2.87 -> 2.83
  // ms); only for the four-wave tiles without VE: the eight-wave ones lost a
  // workgroup per CU (H = 8, D = 32: 0.52 -> 0.62 ms) or spilled (cfg4).
  constexpr bool PP = NW == 4 && !Cfg::VE;
  float4 pjn = PP && use_e && len > 0 ? ra.pos(prm.ev.pos4, min(el % KC, len - 1)) : float4{0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < len; j0 += KC) {
    // ---- VS / KS: stage V[h][key][d] and K (keys past the event are zero) ----
    if constexpr (Cfg::VS) {
      using V16 = typename VecOf<T>::type;
      constexpr int VEC = 16 / Cfg::ESZ;
      constexpr int PER_ROW = D / VEC;
      const int total = H * KC * PER_ROW;
      for (int idx = tid; idx < total; idx += NT) {
        const int dv = idx % PER_ROW;
        const int key = (idx / PER_ROW) % KC;
        const int h = idx / (PER_ROW * KC);
        const int j = j0 + key;
        const long off = rx.off(h, j < len ? j : 0, D) + dv * VEC;
        const V16 val = j < len ? *reinterpret_cast<const V16*>(vg + off) : VecOf<T>::zero();
        *reinterpret_cast<V16*>(Vs + (h * KC + key) * Cfg::V_ROW + dv * VEC) = val;
        if constexpr (Cfg::KS) {
          const V16 kv = j < len ? *reinterpret_cast<const V16*>(kg + off) : VecOf<T>::zero();
          *reinterpret_cast<V16*>(Ks + (h * KC + key) * Cfg::V_ROW + dv * VEC) = kv;
        }
      }
    }

    // ---- row-owner: embedding of its rows x KC keys, then u.E ----
    if (use_e) {
      const int key = el % KC;
      const float4 pj = PP ? pjn : ra.pos(prm.ev.pos4, min(j0 + key, len - 1));
      if (PP && j0 + KC < len) pjn = ra.pos(prm.ev.pos4, min(j0 + KC + key, len - 1));
#pragma unroll
      for (int k2 = 0; k2 < EPL; ++k2) {
        const int il = ws * RW + el / KC + ESTEP * k2;
        write_embedding<T, C, EL::SPLIT>(Es + (il * KC + key) * Cfg::E_ROW, pos_i[k2], pj, prm.freq, epart);
      }
      wave_lds_sync();
      if (attn) {
#pragma unroll
        for (int ri = 0; ri < RW; ++ri) {
          const int il = ws * RW + ri;
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            CFrag<T, C> ef;
            ef.load(Es + (il * KC + 16 * s + n) * Cfg::E_ROW, g);
            const f32x4 ue = mma_c<C>(ef, uf[ri], zero4());
            if (n < H) *reinterpret_cast<f32x4*>(Sf + (il * HP + n) * SLOT_F + 16 * s + 4 * g) = ue;
          }
        }
      }
    }
    __syncthreads();  // V staged; u.E staged

    // ---- head-owner: logits, online softmax, P V ----
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
      const int h = ws * HW + hl;
      if (h >= H) continue;
      // VE: this head's V columns (gathered element by element from clamped
      // keys, zeroed past the event) are loaded before its logits, so they
      // land during the logits product and the softmax.
      JFrag<T, NS> vfe[Cfg::VE ? D / 16 : 1];
      if constexpr (Cfg::VE) {
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
          for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int j = j0 + 16 * s + 4 * g + r;
              const T x = vg[rx.off(h, min(j, len - 1), D) + 16 * dt + n];
              vfe[dt].v[4 * s + r] = j < len ? (float)x : 0.f;
            }
      }
      f32x4 S[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const f32x4 init =
            attn ? *reinterpret_cast<const f32x4*>(Sf + (n * HP + h) * SLOT_F + 16 * s + 4 * g) : zero4();
        KFrag<T, D> kf;
        if constexpr (Cfg::KS) {
          kf.load(Ks + (h * KC + 16 * s + n) * Cfg::V_ROW, g);
        } else {
          int key = j0 + 16 * s + n;
          key = key < len ? key : len - 1;
          kf.load(kg + rx.off(h, key, D), g);
        }
        S[s] = mma_k<D>(kf, qf[hl], init);
      }
      float mx = -INFINITY;
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (j0 + 16 * s + 4 * g + r >= len) S[s][r] = -INFINITY;
          mx = fmaxf(mx, S[s][r]);
        }
      mx = group_allmax(mx);
      const float m_new = fmaxf(m_run[hl], mx);
      const float alpha = exp2f_fast((m_run[hl] - m_new) * kLog2e);
      const float mb = m_new * kLog2e;
      float psum = 0.f;
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pv = exp2f_fast(__builtin_fmaf(S[s][r], kLog2e, -mb));
          S[s][r] = pv;
          psum += pv;
        }
      l_run[hl] = l_run[hl] * alpha + psum;
      m_run[hl] = m_new;
      JFrag<T, NS> pf;
      pf.from_tiles(S);
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        JFrag<T, NS> vf;
        if constexpr (Cfg::VS) {
          vf.load_tr(Vs + h * KC * Cfg::V_ROW, Cfg::V_ROW, 16 * dt, g, n);
        } else if constexpr (Cfg::VE) {
          vf = vfe[dt];
        } else {
#pragma unroll
          for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int j = j0 + 16 * s + 4 * g + r;
              vf.v[4 * s + r] = j < len ? vg[rx.off(h, j, D) + 16 * dt + n] : 0.f;
            }
        }
        O[hl][dt] = mma_j(vf, pf, O[hl][dt] * alpha);
      }
      if (act) {
        // The slot's u.E was consumed above by this wave; P overwrites it.
        wave_lds_sync();
        pf.store_keys(St + (n * HP + h) * SLOT_T, g);
        if (g == 0) As[h * 16 + n] = alpha;
      }
    }
    __syncthreads();  // P and alpha staged; V no longer read

    // ---- row-owner: AE = alpha * AE + E^T P ----
    if (act) {
#pragma unroll
      for (int ri = 0; ri < RW; ++ri) {
        const int il = ws * RW + ri;
        const float alpha = n < H ? As[n * 16 + il] : 1.f;
        JFrag<T, NS> pf;
        if (n < H)
          pf.load_keys(St + (il * HP + n) * SLOT_T, g);
        else
          pf.zero();
#pragma unroll
        for (int ct = 0; ct < C / 16; ++ct) {
          JFrag<T, NS> ef;
          ef.load_tr(Es + il * KC * Cfg::E_ROW, Cfg::E_ROW, 16 * ct, g, n);
          AE[ri][ct] = mma_j(ef, pf, AE[ri][ct] * alpha);
        }
      }
    }
    __syncthreads();  // staging and embedding free for the next chunk
  }

  // ---- epilogue ----
  float inv_l[HW];
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    const float lf = group_allsum(l_run[hl]);
    inv_l[hl] = 1.f / lf;
    const int h = ws * HW + hl;
    if (g == 0 && row_ok && h < H) prm.lse[ra.vec(h, my_row)] = m_run[hl] + logf(lf);
  }

  // One d-tile at a time: the row-owner forms o2^T_i[d, h] = sum_c W[d, c]
  // AE^T_i[c, h] in fp32 MFMA (channel c = 16ct + 4g + s' sits in register
  // s' of lane group g, so step (ct, s') contracts those four) and stages
  // it as [row][head][d]; the head-owner adds it to O and stores
  // out = (O + o2) / l + b.
  T* outg = reinterpret_cast<T*>(prm.out);
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) {
    if (act) {
#pragma unroll
      for (int ri = 0; ri < RW; ++ri) {
        const int il = ws * RW + ri;
        f32x4 acc = zero4();
#pragma unroll
        for (int ct = 0; ct < C / 16; ++ct)
#pragma unroll
          for (int sp = 0; sp < 4; ++sp)
            acc = mfma_f32(prm.weight[(16 * dt + n) * C + 16 * ct + 4 * g + sp], AE[ri][ct][sp], acc);
        if (n < H) *reinterpret_cast<f32x4*>(Sf + (il * HP + n) * SLOT_F + 4 * g) = acc;
      }
      __syncthreads();
    }
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
      const int h = ws * HW + hl;
      if (h >= H) continue;
      f32x4 o = O[hl][dt];
      if (act) o = o + *reinterpret_cast<const f32x4*>(Sf + (n * HP + h) * SLOT_F + 4 * g);
      o = o * inv_l[hl];
      if (act && prm.bias) {
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] += prm.bias[16 * dt + 4 * g + r];
      }
      if (row_ok) store4<T>(outg + ra.off(h, my_row, D) + 16 * dt + 4 * g, o);
    }
    if (act) __syncthreads();
  }

  // Padding rows of this block (and past the event for its last block): 0.
  zero_pad_rows<T>(prm.ev, eb, ra, ra, row0, Cfg::ROWS, D, tid, NT, outg, prm.lse, 1);
}

// ---------------------------------------------------------------------------
// Dispatch. The static choice is the split with the most waves per 16-row
// tile that fits LDS, then 32-key chunks (see pick_split). The plan bits
// FST_PLAN_FWD_T16 / T32 / T64 fix the rows per workgroup (NW = 4, 2, 1) and
// FST_PLAN_FWD_KC16 / KC32 the keys per chunk (NS = 1, 2); a group left
// empty takes the first value in that order that fits with the other.
// Every split computes each (row, head) with the same sequence of
// operations; the key chunk moves the online softmax's rescaling points.
// ---------------------------------------------------------------------------
template <typename T, int HP, int D, int C>
struct FwdPick {
  template <int NW, int NS>
  using F = FwdCfg<T, HP, D, C, NW, NS>;
  // The split for requested (nw, ns) (0: not requested). An eight-wave tile
  // whose waves own two heads or more takes 16-key chunks first (H = 16,
  // D = 32, C = 16, B = 64, L = 768: 0.83 against 1.08 ms; with one head per
  // wave 32-key chunks stay first: cfg4 11.2 against 15.1 ms).
  static constexpr int choose(int nw, int ns) {
    const int s = pick_split<F>(nw, ns);
    return ns == 0 && s / 10 == 8 && HP / 8 >= 2 ? pick_split<F>(8, 0, 1) : s;
  }
  static constexpr int STATIC = choose(0, 0);
  static constexpr int NW = STATIC ? STATIC / 10 : 4, NS = STATIC ? STATIC % 10 : 1;
  using Cfg = F<NW, NS>;
  static constexpr bool OK = STATIC != 0;
  static constexpr int PLANS = OK ? split_plans<F>(FST_PLAN_FWD_T16, FST_PLAN_FWD_KC16, FST_PLAN_FWD_W8) : 0;
};

template <typename T, int HP, int D, int C, int NW, int NS>
int fwd_launch_v(const FwdParams& prm, hipStream_t stream, int grid, bool query, int* rows) {
  using Cfg = FwdCfg<T, HP, D, C, NW, NS>;
  if constexpr (!Cfg::FITS) {
    return FST_EUNSUPPORTED;
  } else {
    *rows = Cfg::ROWS;
    if (query) return FST_OK;
    auto kern = fwd_kernel<T, HP, D, C, NW, NS>;
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::LDS_BYTES) !=
        hipSuccess)
      return FST_ELAUNCH;
    if (grid > 0) hipLaunchKernelGGL(kern, dim3(grid), dim3(Cfg::THREADS), Cfg::LDS_BYTES, stream, prm);
    return hipGetLastError() == hipSuccess ? FST_OK : FST_ELAUNCH;
  }
}

// Launches (or, with query, only checks) the split the plan bits of
// prm.flags name; *rows receives its rows per workgroup.
template <typename T, int HP, int D, int C>
int fwd_launch_t(const FwdParams& prm, hipStream_t stream, int grid, bool query, int* rows) {
  using P = FwdPick<T, HP, D, C>;
  *rows = 0;
  if constexpr (!P::OK) {
    return FST_EUNSUPPORTED;
  } else {
    const int split = P::choose(plan_nw(prm.flags, bit_index(FST_PLAN_FWD_T16), bit_index(FST_PLAN_FWD_W8)),
                                plan_ns(prm.flags, bit_index(FST_PLAN_FWD_KC16)));
    switch (split) {
      case 11: return fwd_launch_v<T, HP, D, C, 1, 1>(prm, stream, grid, query, rows);
      case 12: return fwd_launch_v<T, HP, D, C, 1, 2>(prm, stream, grid, query, rows);
      case 21: return fwd_launch_v<T, HP, D, C, 2, 1>(prm, stream, grid, query, rows);
      case 22: return fwd_launch_v<T, HP, D, C, 2, 2>(prm, stream, grid, query, rows);
      case 41: return fwd_launch_v<T, HP, D, C, 4, 1>(prm, stream, grid, query, rows);
      case 42: return fwd_launch_v<T, HP, D, C, 4, 2>(prm, stream, grid, query, rows);
      case 81: return fwd_launch_v<T, HP, D, C, 8, 1>(prm, stream, grid, query, rows);
      case 82: return fwd_launch_v<T, HP, D, C, 8, 2>(prm, stream, grid, query, rows);
      default: return FST_EUNSUPPORTED;
    }
  }
}

}  // namespace fst
