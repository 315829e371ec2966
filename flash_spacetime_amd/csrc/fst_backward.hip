// Deterministic backward kernels of flash-spacetime attention for gfx950.
//
// Gradients of the spec (reference.py:106-167) in the fused form of
// backward.py:3-32. With qt = q*scale, u = T(qt W), w~ = T(dO W), dob = dO.b:
//   s_ij  = qt_i.k_j + [A] u_i.E_ij,          P_ij = exp(s_ij - lse_i)
//   dP_ij = dO_i.v_j + [V] (w~_i.E_ij + dob_i)
//   D_i   = sum_j P_ij dP_ij / sum_j P_ij   (same P and dP as dS below)
//   dS_ij = P_ij (dP_ij - D_i)
//   dq_i  = scale (sum_j dS_ij k_j + [A] (W sum_j dS_ij E_ij + sigma_i b))
//   dk_j  = sum_i dS_ij qt_i,      dv_j = sum_i P_ij dO_i
//   dW    = [A] sum qt (x) H + [V] sum dO (x) G,   H_i = sum_j dS_ij E_ij,
//           G_i = sum_j P_ij E_ij,  sigma_i = sum_j dS_ij,  db = [V] sum dO
// Forming D from the very P and dP that build dS makes sigma (the row sum of
// dS) vanish by construction (backward.py:371-407); normalising by sum P
// makes it invariant to an O(1) mismatch between the saved LSE and the
// recomputed logits at large logits. The same mismatch scales a row's P by a
// common factor (the forward's fp32 lse of a logit of O(1e4) is rounded to
// ~1e-3), which the gradients would carry: the rows kernel divides its
// accumulators by Z = sum P, and the cols kernel recomputes P / Z with log2 Z
// (lse_z) subtracted after the exponent's fma, where it is not rounded away.
//
// Two kernels, each the single writer of its outputs (no atomics, fixed
// loop order => bitwise deterministic):
//  * rows: workgroups own query rows, same head-owner / row-owner split as
//    the forward. One pass over the keys forms D online (N / Z over the keys
//    seen, the accumulators corrected by the P-sums they lack whenever D
//    moves) and accumulates dq (head-owner), H and G (row-owner), sigma. The
//    epilogue projects H through W into dq, and
//    reduces qt (x) H + dO (x) G and dO over the block's rows into per-block
//    partials of dW and db. u, w~, dob and D go to scratch for the cols
//    kernel.
//  * cols: workgroups own keys and stream query rows -- the forward's
//    structure mirrored (S = Qt K^T with keys on the lanes) -- and
//    accumulate dk and dv. The u.E and w~.E terms of the streamed rows are
//    formed by the pair-owner waves and staged for the head-owners.
//  * a final reduction sums the dW / db block partials in block order.
#include "fst_kernels.h"

namespace fst {

// ---------------------------------------------------------------------------
// Helpers shared by both kernels.
// ---------------------------------------------------------------------------

// One 16-row MFMA tile (rows = the lane index of the C tile's columns) of
// P and dP for one head: s = mma(A_s, B_s) + init_s, dP = mma(A_p, B_p) +
// init_p, both already computed by the caller; this applies masking, the
// exponential and the dob term. Written once and used by both kernels so
// the arithmetic of P and dP is identical wherever they are recomputed.
__device__ __forceinline__ void finish_p_dp(f32x4& s, f32x4& dp, float lse2, float dob, unsigned valid_mask) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const bool ok = (valid_mask >> r) & 1u;
    const float p = exp2f_fast(__builtin_fmaf(s[r], kLog2e, -lse2));
    s[r] = ok ? p : 0.f;
    dp[r] = dp[r] + dob;
  }
}

// ---------------------------------------------------------------------------
// Rows kernel.
// ---------------------------------------------------------------------------
template <typename T, int HP, int D, int C, int NW, int NS>
struct BwdRowsCfg {
  static constexpr bool BF = is_bf16<T>::value;
  static constexpr int HW = HP / NW, RW = 16 / NW;
  static constexpr int WPG = NW > 4 ? NW : 4, THREADS = 64 * WPG;  // waves, threads per workgroup
  static constexpr int TILES = WPG / NW, ROWS = 16 * TILES;
  static constexpr int KC = 16 * NS;
  static constexpr int ESZ = sizeof(T);
  static constexpr int PAD = 16 / ESZ;
  static constexpr int KV_ROW = D + PAD;
  static constexpr int DW_BYTES = 4 * (D * C + D) * 4;                  // dW/db partials of four waves
  static constexpr int E_ROW = C + PAD;
  static constexpr int E_TILE = 16 * KC * E_ROW * ESZ;
  static constexpr int U_ROW = KC + 4;   // fp32 per staged u.E / w~.E
  static constexpr int P_ROW = KC + PAD; // T per staged P / dS
  static constexpr int SLOT_A = 2 * U_ROW * 4;
  static constexpr int SLOT_B = 2 * P_ROW * ESZ;
  static constexpr int SLOT_O = 20 * 4;
  static constexpr int SLOT_HG = 2 * 20 * 4;  // one 16-channel tile of H and G
  static constexpr int SLOT_1 = SLOT_A > SLOT_B ? SLOT_A : SLOT_B;
  static constexpr int SLOT_2 = SLOT_O > SLOT_HG ? SLOT_O : SLOT_HG;
  static constexpr int SLOT = SLOT_1 > SLOT_2 ? SLOT_1 : SLOT_2;
  static constexpr int STAGE_TILE = 16 * HP * SLOT;
  static constexpr int DD_BYTES = 16 * HP * 4;  // per (row, head) increments of D
  static constexpr int TILE_BYTES = E_TILE + STAGE_TILE + DD_BYTES;
  // KVS: each chunk's K and V rows are staged in LDS by the whole workgroup
  // (coalesced 16-byte loads, then row fragments and transposed K read back
  // from LDS); bf16 only. For float32 every head-owner wave loads its K and
  // V fragments from global memory instead: staged, the float32 kernel was
  // slower on gfx950 (cfg4: 45.7 against 41.2 ms; B=256 L=768 H=12 D=32
  // C=16: 10.6 against 9.7 ms), its synchronous staging serialising what
  // the waves' own loads overlap.
  static constexpr int KV_STAGED = 2 * HP * KC * KV_ROW * ESZ;
  static constexpr bool KVS = BF;
  static constexpr int KV_BYTES = KVS ? KV_STAGED : 0;                 // K and V
  static constexpr int R0_BYTES = KV_BYTES > DW_BYTES ? KV_BYTES : DW_BYTES;
  static constexpr int LDS_BYTES = R0_BYTES + TILES * TILE_BYTES;
  // UL (float32): the row-owner's u and w~ fragments (C values per row and
  // head) live in region R0 during the key loop instead of registers; R0
  // holds the dW reduction only after the loop. Where it fits (HP = 8, D = C
  // = 64: 64 KB of R0's 66.5) it frees C / 2 VGPRs per row of a wave (64 at
  // cfg4's two rows per wave).
  static constexpr int UW_BYTES = 2 * ROWS * HP * C * 4;
  static constexpr bool UL = !BF && !KVS && UW_BYTES <= R0_BYTES;
  // KE (K from global memory): a chunk's transposed K (the dQ product's
  // operand, gathered element by element) is loaded at the start of the
  // chunk, so it lands during the row-owner part instead of being waited for
  // by the head-owner (B=256 L=768 H=12 D=32 C=16 in float32: rows kernel
  // 6.38 -> 6.08 ms; cfg4 20.07 -> 19.66 ms). Issuing the K and V row
  // fragments early as well measured slower there (6.47 ms) and needs three
  // times the registers. It holds HW D / 4 more registers per lane over the
  // row-owner part: on for the static splits (16-key chunks; eight waves, or
  // four where 8 does not divide HP) where the lane-state estimate (HP / NW)
  // D + (16 / NW) C plus those stays within what compiled without new
  // spills on gfx950: 148 with eight waves (256 registers per lane), 244
  // (one pass) or 312 (two passes) with four (512); and for cfg4's split
  // (eight waves of one head, u / w~ in LDS), faster although it spills
  // three registers.
  static constexpr int KE_STATE = HW * D + RW * C + HW * D / 4;
  template <int PASSES>
  static constexpr bool ke() {
    return !KVS && NS == 1 &&
           (NW == 8 ? KE_STATE <= 148 || (UL && HW == 1)
                    : NW == 4 && HP % 8 != 0 ? KE_STATE <= (PASSES == 1 ? 244 : 312) : false);
  }
  // A row-owner wave's RW rows x KC keys: whole embeddings per lane, or
  // whole groups of four frequencies per lane where lanes share a pair.
  using EL = EmbedLanes<RW * KC>;
  static constexpr bool FITS = LDS_BYTES <= 160 * 1024 && HP % NW == 0 && EL::OK && (C / 2 / EL::SPLIT) % 4 == 0;
  static_assert(SLOT % 16 == 0, "slot alignment");
};

// PASSES = 1: one pass over the keys with D formed online; 2: a first pass
// forms D, the second accumulates with it (no corrections, no sum P k, H
// and G live only in the second pass: fewer registers at the large
// layouts).
template <typename T, int HP, int D, int C, int NW, int NS, int PASSES>
__global__ __launch_bounds__(64 * (NW > 4 ? NW : 4), 1) void bwd_rows_kernel(BwdParams prm) {
  using Cfg = BwdRowsCfg<T, HP, D, C, NW, NS>;
  constexpr int NT = Cfg::THREADS;
  constexpr bool BF = Cfg::BF;
  constexpr bool KE = Cfg::template ke<PASSES>();
  constexpr int HW = Cfg::HW, RW = Cfg::RW, KC = Cfg::KC;
  constexpr int SLOT_F = Cfg::SLOT / 4, SLOT_T = Cfg::SLOT / Cfg::ESZ;
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int tile = wave / NW, ws = wave % NW;

  EventBlock eb;
  if (!locate_block(prm.ev, blockIdx.x, eb)) return;
  const int len = eb.len;
  const int H = prm.H;
  const bool attn = prm.flags & FST_ATTN_BIAS;
  const bool act = prm.flags & FST_ACT_BIAS;
  const bool use_e = attn || act;
  const bool use_b = act && prm.bias;
  const RowAddr ra = row_addr(prm.ev, eb);   // dO, lse, dob, D, rowsum, u, w~
  const RowAddr rx = row_addr_x(prm.ev, eb);  // q, k, v, dq
  const int row0 = eb.blk * Cfg::ROWS;
  const int i0 = row0 + 16 * tile;
  if (event_refused(prm.ev, eb)) {
    fill_rows_nan<T, D>(rx, ra, row0, min(row0 + Cfg::ROWS, len), H, tid, NT, reinterpret_cast<T*>(prm.dq),
                        prm.rowsum);
    float* part = prm.dw_part + (long)blockIdx.x * (D * C + D);
    for (int e = tid; e < D * C + D; e += NT) part[e] = __builtin_nanf("");
    return;
  }

  T* Ks = reinterpret_cast<T*>(smem);
  T* Vs = Ks + HP * KC * Cfg::KV_ROW;
  float* Wred = reinterpret_cast<float*>(smem);  // epilogue: [4][D*C + D], one slot per wave mod 4
  unsigned char* tbase = smem + Cfg::R0_BYTES + tile * Cfg::TILE_BYTES;
  T* Es = reinterpret_cast<T*>(tbase);
  float* Sf = reinterpret_cast<float*>(tbase + Cfg::E_TILE);
  T* St = reinterpret_cast<T*>(tbase + Cfg::E_TILE);
  float* Dd = reinterpret_cast<float*>(tbase + Cfg::E_TILE + Cfg::STAGE_TILE);  // [HP][16] increments of D

  const T* __restrict__ qg = reinterpret_cast<const T*>(prm.q);
  const T* __restrict__ kg = reinterpret_cast<const T*>(prm.k);
  const T* __restrict__ vg = reinterpret_cast<const T*>(prm.v);
  const T* __restrict__ dog = reinterpret_cast<const T*>(prm.dout);

  // ---- head-owner state (rows on lane n) ----
  // PASSES = 1: one pass over the keys. D = N / Z is formed online: after chunk t the
  // running D_t (N, Z over the keys seen) replaces D_{t-1}, and the
  // accumulators built with the old value are corrected with the P-sums
  // they lack (dQ -= dD A2, A2 = sum P k; H -= dD G; sigma -= dD Z), so at
  // the end each equals its two-pass value for D = N / Z over all keys
  // (backward.py:371-407 forms D in a first pass). sigma is the sum of the
  // dS values the products were fed, with the same corrections.
  const int my_row = i0 + n;
  const bool row_ok = my_row < len;
  KFrag<T, D> qf[HW], dof[HW];
  f32x4 dQ[HW][D / 16], A2[HW][D / 16];
  float lse2[HW], dobv[HW], nsum[HW], zsum[HW], dval[HW], sig[HW], zlane[HW];
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    const int h = ws * HW + hl;
    const bool ok = h < H && row_ok;
    if (ok) {
      qf[hl].load_scaled(qg + rx.off(h, my_row, D), g, prm.scale);
      dof[hl].load(dog + ra.off(h, my_row, D), g);
    } else {
      qf[hl].zero();
      dof[hl].zero();
    }
    lse2[hl] = ok ? prm.lse[ra.vec(h, my_row)] * kLog2e : 0.f;
    // dob = dO . b in fp32 (backward.py:548-552): each lane group holds a
    // quarter of the row; the four partial sums are combined.
    float part = 0.f;
    if (use_b && ok) {
      const T* dp = dog + ra.off(h, my_row, D);
#pragma unroll
      for (int d4 = 0; d4 < D / 4; ++d4) {
        const int d = (D / 4) * g + d4;
        part = __builtin_fmaf((float)dp[d], prm.bias[d], part);
      }
    }
    dobv[hl] = group_allsum(part);
    if (g == 0 && ok) prm.dob[ra.vec(h, my_row)] = dobv[hl];
    nsum[hl] = zsum[hl] = sig[hl] = dval[hl] = zlane[hl] = 0.f;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) dQ[hl][dt] = A2[hl][dt] = zero4();
  }

  // ---- row-owner state (heads on lane n) ----
  CFrag<T, C> uf[RW], wf[RW];
  f32x4 Hacc[RW][C / 16], Gacc[RW][C / 16];
  T* __restrict__ ug = reinterpret_cast<T*>(prm.u);
  T* __restrict__ wg_ = reinterpret_cast<T*>(prm.wt);
#pragma unroll
  for (int ri = 0; ri < RW; ++ri) {
    const int row = i0 + ws * RW + ri;
    const bool ok = row < len && n < H;
    f32x4 acc[C / 16];
    if (attn) {
      project_row<T, D, C>(qg + rx.off(0, ok ? row : 0, D), rx.hs * D, ok, prm.scale, prm.weight, g, n, acc);
      uf[ri].from_acc(acc);
      if (ok)
#pragma unroll
        for (int ct = 0; ct < C / 16; ++ct) {
          f32x4 rq;
#pragma unroll
          for (int r = 0; r < 4; ++r) rq[r] = (float)(T)acc[ct][r];
          store4<T>(ug + ra.off(n, row, C) + 16 * ct + 4 * g, rq);
        }
    } else {
      uf[ri].zero();
    }
    if (act) {
      project_row<T, D, C>(dog + ra.off(0, ok ? row : 0, D), ra.hs * D, ok, 1.f, prm.weight, g, n, acc);
      wf[ri].from_acc(acc);
      if (ok)
#pragma unroll
        for (int ct = 0; ct < C / 16; ++ct) {
          f32x4 rq;
#pragma unroll
          for (int r = 0; r < 4; ++r) rq[r] = (float)(T)acc[ct][r];
          store4<T>(wg_ + ra.off(n, row, C) + 16 * ct + 4 * g, rq);
        }
    } else {
      wf[ri].zero();
    }
#pragma unroll
    for (int ct = 0; ct < C / 16; ++ct) Hacc[ri][ct] = Gacc[ri][ct] = zero4();
  }
  // UL: [u, w~][row of the workgroup][channel tile][lane group][head] f32x4,
  // written and read by the row's own wave. Lanes of padded heads (n >= HP)
  // read head HP - 1's slot: they only feed output columns that are never
  // stored.
  float* Ul = reinterpret_cast<float*>(smem);
  const int hn = n < HP ? n : HP - 1;
  auto ul_off = [&](int op, int ri, int ct) {
    const int il = 16 * tile + ws * RW + ri;
    return ((((op * Cfg::ROWS + il) * (C / 16) + ct) * 4 + g) * HP + hn) * 4;
  };
  if constexpr (Cfg::UL) {
#pragma unroll
    for (int ri = 0; ri < RW; ++ri)
#pragma unroll
      for (int ct = 0; ct < C / 16; ++ct)
        if (n < HP) {
          *reinterpret_cast<f32x4*>(Ul + ul_off(0, ri, ct)) = uf[ri].v[ct];
          *reinterpret_cast<f32x4*>(Ul + ul_off(1, ri, ct)) = wf[ri].v[ct];
        }
    wave_lds_sync();
  }
  auto row_frag = [&](int op, int ri) __attribute__((always_inline)) {
    if constexpr (Cfg::UL) {
      CFrag<T, C> f;
#pragma unroll
      for (int ct = 0; ct < C / 16; ++ct) f.v[ct] = *reinterpret_cast<const f32x4*>(Ul + ul_off(op, ri, ct));
      return f;
    } else {
      return op == 0 ? uf[ri] : wf[ri];
    }
  };
  using EL = typename Cfg::EL;  // lane slot el -> key el % KC, rows el / KC + (64 / KC) k2
  constexpr int EPL = EL::EPL;
  constexpr int ESTEP = 64 / KC;
  const int el = EL::slot(lane), epart = EL::part(lane);
  float4 pos_i[EPL];
#pragma unroll
  for (int k2 = 0; k2 < EPL; ++k2) {
    const int row = i0 + ws * RW + el / KC + ESTEP * k2;
    pos_i[k2] = use_e ? ra.pos(prm.ev.pos4, row < len ? row : (len > 0 ? len - 1 : 0)) : float4{0.f, 0.f, 0.f, 0.f};
  }

  // Key positions run a chunk ahead (the next pass's first chunk after the
  // last): the embedding needs them first thing in a chunk (B=256 L=768 H=12
  // D=32 C=16 in float32: 6.06 -> 5.67 ms; cfg4 19.69 -> 19.27 ms).
  float4 pjn = use_e && len > 0 ? ra.pos(prm.ev.pos4, min(el % KC, len - 1)) : float4{0.f, 0.f, 0.f, 0.f};
  for (int pass = 0; pass < PASSES; ++pass) {
    for (int j0 = 0; j0 < len; j0 += KC) {
      // ---- KVS: stage K and V rows of the chunk (zero past the event) ----
      if constexpr (Cfg::KVS) {
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
          const V16 kv = j < len ? *reinterpret_cast<const V16*>(kg + off) : VecOf<T>::zero();
          const V16 vv = j < len ? *reinterpret_cast<const V16*>(vg + off) : VecOf<T>::zero();
          *reinterpret_cast<V16*>(Ks + (h * KC + key) * Cfg::KV_ROW + dv * VEC) = kv;
          *reinterpret_cast<V16*>(Vs + (h * KC + key) * Cfg::KV_ROW + dv * VEC) = vv;
        }
      }
      // ---- KE: the head-owner's transposed K of the chunk, loaded from
      // clamped keys (padded heads read head H - 1) and zeroed past the
      // event after the load ----
      constexpr int KH = KE ? HW : 1;
      JFrag<T, NS> kte[KH][D / 16];
      if constexpr (KE) {
#pragma unroll
        for (int hl = 0; hl < HW; ++hl) {
          const int hc = min(ws * HW + hl, H - 1);
#pragma unroll
          for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
            for (int s = 0; s < NS; ++s)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int j = j0 + 16 * s + 4 * g + r;
                const T x = kg[rx.off(hc, min(j, len - 1), D) + 16 * dt + n];
                kte[hl][dt].v[4 * s + r] = j < len ? (float)x : 0.f;
              }
        }
      }
      // ---- row-owner: embedding, u.E and w~.E staged per (row, head) ----
      if (use_e) {
        const int key = el % KC;
        const float4 pj = pjn;
        pjn = ra.pos(prm.ev.pos4, min((j0 + KC < len ? j0 + KC : 0) + key, len - 1));
#pragma unroll
        for (int k2 = 0; k2 < EPL; ++k2) {
          const int il = ws * RW + el / KC + ESTEP * k2;
          write_embedding<T, C, EL::SPLIT>(Es + (il * KC + key) * Cfg::E_ROW, pos_i[k2], pj, prm.freq, epart);
        }
        wave_lds_sync();
#pragma unroll
        for (int ri = 0; ri < RW; ++ri) {
          const int il = ws * RW + ri;
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            CFrag<T, C> ef;
            ef.load(Es + (il * KC + 16 * s + n) * Cfg::E_ROW, g);
            float* slot = Sf + (il * HP + n) * SLOT_F;
            if (attn) {
              const f32x4 ue = mma_c<C>(ef, row_frag(0, ri), zero4());
              if (n < H) *reinterpret_cast<f32x4*>(slot + 16 * s + 4 * g) = ue;
            }
            if (act) {
              const f32x4 we = mma_c<C>(ef, row_frag(1, ri), zero4());
              if (n < H) *reinterpret_cast<f32x4*>(slot + Cfg::U_ROW + 16 * s + 4 * g) = we;
            }
          }
        }
      }
      __syncthreads();

      // ---- head-owner: P, dP, online D, dS, dQ ----
#pragma unroll
      for (int hl = 0; hl < HW; ++hl) {
        const int h = ws * HW + hl;
        if (h >= H) continue;
        f32x4 S[NS], P_[NS];
        const float* slot = Sf + (n * HP + h) * SLOT_F;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const f32x4 ue = attn ? *reinterpret_cast<const f32x4*>(slot + 16 * s + 4 * g) : zero4();
          const f32x4 we = act ? *reinterpret_cast<const f32x4*>(slot + Cfg::U_ROW + 16 * s + 4 * g) : zero4();
          KFrag<T, D> kf, vf;
          if constexpr (Cfg::KVS) {
            kf.load(Ks + (h * KC + 16 * s + n) * Cfg::KV_ROW, g);
            vf.load(Vs + (h * KC + 16 * s + n) * Cfg::KV_ROW, g);
          } else {
            const int key = min(j0 + 16 * s + n, len - 1);
            kf.load(kg + rx.off(h, key, D), g);
            vf.load(vg + rx.off(h, key, D), g);
          }
          S[s] = mma_k<D>(kf, qf[hl], ue);
          P_[s] = mma_k<D>(vf, dof[hl], we);
          unsigned vm = 0;
#pragma unroll
          for (int r = 0; r < 4; ++r) vm |= (j0 + 16 * s + 4 * g + r < len ? 1u : 0u) << r;
          finish_p_dp(S[s], P_[s], lse2[hl], dobv[hl], vm);
        }
        // S now holds P, P_ holds dP.
        float nt = 0.f, zt = 0.f;
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            nt = __builtin_fmaf(S[s][r], P_[s][r], nt);
            zt += S[s][r];
          }
        float dD = 0.f;
        if constexpr (PASSES == 2) {
          if (pass == 0) {  // the first pass forms N and Z only
            group_allsum2(nt, zt);
            nsum[hl] += nt;
            zsum[hl] += zt;
            continue;
          }
        } else {
          float ns = nt, zs = zt;  // zt stays this lane's part
          group_allsum2(ns, zs);
          nsum[hl] += ns;
          zsum[hl] += zs;
          const float dn = zsum[hl] > 0.f ? nsum[hl] / zsum[hl] : 0.f;
          dD = dn - dval[hl];
          dval[hl] = dn;
          sig[hl] = __builtin_fmaf(-dD, zlane[hl], sig[hl]);
          zlane[hl] += zt;
        }
        {
          f32x4 dS[NS];
          {
            // sigma sums the rounded dS the products are fed: no fused
            // multiply-add here, whatever the surrounding code's layout (the
            // compiler's fusing otherwise differed between plan variants).
#pragma clang fp contract(off)
#pragma unroll
            for (int s = 0; s < NS; ++s)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                dS[s][r] = S[s][r] * (P_[s][r] - dval[hl]);
                sig[hl] += dS[s][r];
              }
          }
          JFrag<T, NS> dsf, pf;
          dsf.from_tiles(dS);
          pf.from_tiles(S);
#pragma unroll
          for (int dt = 0; dt < D / 16; ++dt) {
            JFrag<T, NS> kt;
            if constexpr (Cfg::KVS) {
              kt.load_tr(Ks + h * KC * Cfg::KV_ROW, Cfg::KV_ROW, 16 * dt, g, n);
            } else if constexpr (KE) {
              kt = kte[hl][dt];
            } else {
#pragma unroll
              for (int s = 0; s < NS; ++s)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const int j = j0 + 16 * s + 4 * g + r;
                  kt.v[4 * s + r] = j < len ? kg[rx.off(h, j, D) + 16 * dt + n] : 0.f;
                }
            }
            if constexpr (PASSES == 1) {
              dQ[hl][dt] = dQ[hl][dt] - dD * A2[hl][dt];
              A2[hl][dt] = mma_j(kt, pf, A2[hl][dt]);
            }
            dQ[hl][dt] = mma_j(kt, dsf, dQ[hl][dt]);
          }
          if (use_e) {
            wave_lds_sync();  // the slot's u.E / w~.E were read above
            T* tslot = St + (n * HP + h) * SLOT_T;
            pf.store_keys(tslot, g);
            dsf.store_keys(tslot + Cfg::P_ROW, g);
            if (PASSES == 1 && g == 0) Dd[h * 16 + n] = dD;
          }
        }
      }
      __syncthreads();

      // ---- row-owner: H -= dD G; H += E^T dS, G += E^T P (last pass) ----
      if (use_e && pass == PASSES - 1) {
#pragma unroll
        for (int ri = 0; ri < RW; ++ri) {
          const int il = ws * RW + ri;
          const float dd = (PASSES == 1 && n < H) ? Dd[n * 16 + il] : 0.f;
          JFrag<T, NS> pf, dsf;
          if (n < H) {
            const T* tslot = St + (il * HP + n) * SLOT_T;
            pf.load_keys(tslot, g);
            dsf.load_keys(tslot + Cfg::P_ROW, g);
          } else {
            pf.zero();
            dsf.zero();
          }
#pragma unroll
          for (int ct = 0; ct < C / 16; ++ct) {
            JFrag<T, NS> ef;
            ef.load_tr(Es + il * KC * Cfg::E_ROW, Cfg::E_ROW, 16 * ct, g, n);
            if (attn) {
              if constexpr (PASSES == 1) Hacc[ri][ct] = Hacc[ri][ct] - dd * Gacc[ri][ct];
              Hacc[ri][ct] = mma_j(ef, dsf, Hacc[ri][ct]);
            }
            // G also feeds H's corrections in the one-pass form.
            if (PASSES == 1 || act) Gacc[ri][ct] = mma_j(ef, pf, Gacc[ri][ct]);
          }
        }
      }
      __syncthreads();
    }
    if (PASSES == 2 && pass == 0) {
#pragma unroll
      for (int hl = 0; hl < HW; ++hl) dval[hl] = zsum[hl] > 0.f ? nsum[hl] / zsum[hl] : 0.f;
    }
  }
  // P / Z: every accumulator divided by the row's Z (dQ and sigma here, H
  // and G through the per-tile D slots, free after the key loop).
  float rz[HW];
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    const int h = ws * HW + hl;
    rz[hl] = zsum[hl] > 0.f ? 1.f / zsum[hl] : 1.f;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) dQ[hl][dt] = dQ[hl][dt] * rz[hl];
    if (g == 0 && h < H && row_ok) {
      prm.dsum[ra.vec(h, my_row)] = dval[hl];
      prm.lse_z[ra.vec(h, my_row)] = zsum[hl] > 0.f ? log2f(zsum[hl]) : 0.f;
    }
    if (use_e && g == 0) Dd[h * 16 + n] = rz[hl];
  }
  if (use_e) {
    __syncthreads();
#pragma unroll
    for (int ri = 0; ri < RW; ++ri) {
      const float zr = n < H ? Dd[n * 16 + ws * RW + ri] : 1.f;
#pragma unroll
      for (int ct = 0; ct < C / 16; ++ct) {
        Hacc[ri][ct] = Hacc[ri][ct] * zr;
        Gacc[ri][ct] = Gacc[ri][ct] * zr;
      }
    }
  }

  // ---- epilogue: dq = scale (dQ + W H + sigma b) ----
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    sig[hl] = group_allsum(sig[hl]) * rz[hl];
    const int h = ws * HW + hl;
    if (prm.rowsum && g == 0 && h < H && row_ok) prm.rowsum[ra.vec(h, my_row)] = sig[hl];
  }
  T* dqg = reinterpret_cast<T*>(prm.dq);
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) {
    if (attn) {
#pragma unroll
      for (int ri = 0; ri < RW; ++ri) {
        const int il = ws * RW + ri;
        f32x4 acc = zero4();
#pragma unroll
        for (int ct = 0; ct < C / 16; ++ct)
#pragma unroll
          for (int sp = 0; sp < 4; ++sp)
            acc = mfma_f32(prm.weight[(16 * dt + n) * C + 16 * ct + 4 * g + sp], Hacc[ri][ct][sp], acc);
        if (n < H) *reinterpret_cast<f32x4*>(Sf + (il * HP + n) * SLOT_F + 4 * g) = acc;
      }
      __syncthreads();
    }
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
      const int h = ws * HW + hl;
      if (h >= H) continue;
      f32x4 o = dQ[hl][dt];
      if (attn) {
        o = o + *reinterpret_cast<const f32x4*>(Sf + (n * HP + h) * SLOT_F + 4 * g);
        if (prm.bias) {
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = __builtin_fmaf(sig[hl], prm.bias[16 * dt + 4 * g + r], o[r]);
        }
      }
      o = o * prm.scale;
      if (row_ok) store4<T>(dqg + rx.off(h, my_row, D) + 16 * dt + 4 * g, o);
    }
    if (attn) __syncthreads();
  }

  // ---- dW / db partials of this block: sum over its rows and heads ----
  if (use_e) {
    // dW[d, c] += sum_(row, head) A[d, (row, head)] B[(row, head), c] on fp32
    // MFMA: a step covers heads 4s + g of one row; A = qt (resp. dO) with d
    // on the lanes, B = H (resp. G) with c on the lanes, read back from LDS
    // one 16-channel tile at a time as [row][head][c].
    f32x4 dw[D / 16][C / 16];
    float dbl[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
      dbl[dt] = 0.f;
#pragma unroll
      for (int ct = 0; ct < C / 16; ++ct) dw[dt][ct] = zero4();
    }
#pragma unroll
    for (int ct = 0; ct < C / 16; ++ct) {
#pragma unroll
      for (int ri = 0; ri < RW; ++ri) {
        const int il = ws * RW + ri;
        float* slot = Sf + (il * HP + n) * SLOT_F;
        if (n < H) {
          *reinterpret_cast<f32x4*>(slot + 4 * g) = Hacc[ri][ct];
          *reinterpret_cast<f32x4*>(slot + 20 + 4 * g) = Gacc[ri][ct];
        }
      }
      __syncthreads();
#pragma unroll
      for (int ri = 0; ri < RW; ++ri) {
        const int il = ws * RW + ri;
        const int row = i0 + il;
        const bool rok = row < len;
#pragma unroll
        for (int s4 = 0; s4 < HP / 4; ++s4) {
          const int h = 4 * s4 + g;
          const bool ok = rok && h < H;
          const float* slot = Sf + (il * HP + h) * SLOT_F;
          const float bh = (attn && ok) ? slot[n] : 0.f;
          const float bg = (act && ok) ? slot[20 + n] : 0.f;
#pragma unroll
          for (int dt = 0; dt < D / 16; ++dt) {
            const int d = 16 * dt + n;
            const float aq = (attn && ok) ? (float)qg[rx.off(h, row, D) + d] * prm.scale : 0.f;
            const float ao = (act && ok) ? (float)dog[ra.off(h, row, D) + d] : 0.f;
            if (ct == 0) dbl[dt] += ao;
            dw[dt][ct] = mfma_f32(aq, bh, dw[dt][ct]);
            dw[dt][ct] = mfma_f32(ao, bg, dw[dt][ct]);
          }
        }
      }
      __syncthreads();
    }
    // Eight waves: waves 4-7 store their partials first, waves 0-3 add
    // theirs to the slot of the same index (a fixed order).
    float* wr = Wred + (wave & 3) * (D * C + D);
    float dbs[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) dbs[dt] = group_allsum(dbl[dt]);
#pragma unroll
    for (int round = Cfg::WPG / 4 - 1; round >= 0; --round) {
      if (wave >> 2 == round) {
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
#pragma unroll
          for (int ct = 0; ct < C / 16; ++ct)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float* dst = wr + (16 * dt + 4 * g + r) * C + 16 * ct + n;
              *dst = round == Cfg::WPG / 4 - 1 ? dw[dt][ct][r] : *dst + dw[dt][ct][r];
            }
          float* dst = wr + D * C + 16 * dt + n;
          if (g == 0) *dst = round == Cfg::WPG / 4 - 1 ? dbs[dt] : *dst + dbs[dt];
        }
      }
      __syncthreads();
    }
    float* part = prm.dw_part + (long)blockIdx.x * (D * C + D);
    for (int e = tid; e < D * C + D; e += NT) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) acc += Wred[w * (D * C + D) + e];
      part[e] = acc;
    }
  }

  zero_pad_rows<T>(prm.ev, eb, rx, ra, row0, Cfg::ROWS, D, tid, NT, dqg, prm.rowsum, 1);
}

// ---------------------------------------------------------------------------
// Cols kernel: keys owned (lanes), query rows streamed in chunks of KC.
// ---------------------------------------------------------------------------
template <typename T, int HP, int D, int C, int NW, int NS>
struct BwdColsCfg {
  static constexpr bool BF = is_bf16<T>::value;
  static constexpr int HW = HP / NW;
  static constexpr int WPG = NW > 4 ? NW : 4, THREADS = 64 * WPG;  // waves, threads per workgroup
  static constexpr int TILES = WPG / NW, KEYS = 16 * TILES;
  static constexpr int KC = 16 * NS;          // streamed rows per chunk
  static constexpr int RWS = KC / NW;         // streamed rows per pair-owner wave
  static constexpr int ESZ = sizeof(T);
  static constexpr int PAD = 16 / ESZ;
  static constexpr int QO_ROW = D + PAD;
  static constexpr int VEC_BYTES = 4 * HP * KC * 4;                     // lse2, D, dob, log2 Z
  static constexpr int E_ROW = C + PAD;
  static constexpr int E_TILE = KC * 16 * E_ROW * ESZ;                   // [row][key][c]
  static constexpr int UW_ROW = KC + 4;                                 // fp32 rows per (head, key)
  static constexpr int UW_TILE = 2 * HP * 16 * UW_ROW * 4;              // u.E and w~.E
  static constexpr int TILE_BYTES = E_TILE + UW_TILE;
  // QOS: each chunk's qt (= q * scale) and dO rows are staged in LDS by the
  // whole workgroup: always for bf16, for float32 wherever the staged plan
  // fits (the transposed operands are otherwise gathered element by element
  // from global memory; staged, cfg4's float32 cols kernel took 30.7 against
  // 33.1 ms and B=256 L=768 H=12 D=32 C=16's 8.39 against 9.02 ms).
  static constexpr int QO_STAGED = 2 * HP * KC * QO_ROW * ESZ;
  static constexpr bool QOS = BF || QO_STAGED + VEC_BYTES + TILES * TILE_BYTES <= 160 * 1024;
  static constexpr int QO_BYTES = QOS ? QO_STAGED : 0;  // qt and dO
  static constexpr int LDS_BYTES = QO_BYTES + VEC_BYTES + TILES * TILE_BYTES;
  // ER (float32, C a multiple of 32, HP <= 8): the pair-owner forms E in
  // registers in the products' operand layout (embed_cfrag) instead of
  // through LDS, and its rows' u and w~ go straight to the E tile's LDS
  // (wave-private [row][u, w~][head][C + 4] blocks, loaded by direct loads
  // issued a phase ahead) instead of being loaded from global memory where
  // they are used. The blocks take 2 HP / 16 of the E tile.
  static constexpr int UWL_ROW = (C + 4) * 4;                 // bytes per (row, op, head)
  static constexpr int UWL_SLOTS = HP * UWL_ROW / 16;         // 16-byte slots per (row, op)
  static constexpr int UWL_LOADS = (UWL_SLOTS + 63) / 64;     // direct loads per (row, op)
  static constexpr bool ER = !BF && C % 32 == 0 && TILES == 1 && 2 * HP <= 16;
  // The pair-owner's RWS rows x 16 keys: whole embeddings per lane, or
  // whole groups of four frequencies per lane where lanes share a pair.
  using EL = EmbedLanes<RWS * 16>;
  static constexpr bool FITS =
      LDS_BYTES <= 160 * 1024 && HP % NW == 0 && RWS >= 1 && EL::OK && (C / 2 / EL::SPLIT) % 4 == 0;
};

template <typename T, int HP, int D, int C, int NW, int NS>
__global__ __launch_bounds__(64 * (NW > 4 ? NW : 4), 1) void bwd_cols_kernel(BwdParams prm) {
  using Cfg = BwdColsCfg<T, HP, D, C, NW, NS>;
  constexpr int NT = Cfg::THREADS;
  constexpr bool BF = Cfg::BF;
  constexpr int HW = Cfg::HW, KC = Cfg::KC, RWS = Cfg::RWS;
  constexpr int UWR = Cfg::UW_ROW;
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int tile = wave / NW, ws = wave % NW;

  EventSpec ev = prm.ev;
  ev.blkcum = prm.blkcum_cols;
  EventBlock eb;
  if (!locate_block(ev, blockIdx.x, eb)) return;
  const int len = eb.len;
  const int H = prm.H;
  const bool attn = prm.flags & FST_ATTN_BIAS;
  const bool act = prm.flags & FST_ACT_BIAS;
  const bool use_e = attn || act;
  const RowAddr ra = row_addr(ev, eb);   // dO, lse, dob, D, u, w~
  const RowAddr rx = row_addr_x(ev, eb);  // q, k, v, dk, dv
  const int key0 = eb.blk * Cfg::KEYS;
  const int j0t = key0 + 16 * tile;
  if (event_refused(ev, eb)) {
    fill_rows_nan<T, D>(rx, rx, key0, min(key0 + Cfg::KEYS, len), H, tid, NT, reinterpret_cast<T*>(prm.dk), nullptr);
    fill_rows_nan<T, D>(rx, rx, key0, min(key0 + Cfg::KEYS, len), H, tid, NT, reinterpret_cast<T*>(prm.dv), nullptr);
    return;
  }

  T* Qs = reinterpret_cast<T*>(smem);                 // [HP][KC][QO_ROW] T(q*scale)
  T* Os = Qs + HP * KC * Cfg::QO_ROW;                 // [HP][KC][QO_ROW] dO
  float* Lv = reinterpret_cast<float*>(smem + Cfg::QO_BYTES);  // [4][HP][KC]
  unsigned char* tbase = smem + Cfg::QO_BYTES + Cfg::VEC_BYTES + tile * Cfg::TILE_BYTES;
  T* Es = reinterpret_cast<T*>(tbase);                               // [KC][16][E_ROW]
  float* UWs = reinterpret_cast<float*>(tbase + Cfg::E_TILE);        // [2][HP][16][UW_ROW]

  const T* __restrict__ qg = reinterpret_cast<const T*>(prm.q);
  const T* __restrict__ kg = reinterpret_cast<const T*>(prm.k);
  const T* __restrict__ vg = reinterpret_cast<const T*>(prm.v);
  const T* __restrict__ dog = reinterpret_cast<const T*>(prm.dout);
  const T* __restrict__ ug = reinterpret_cast<const T*>(prm.u);
  const T* __restrict__ wg_ = reinterpret_cast<const T*>(prm.wt);

  // ---- head-owner: own keys on lane n ----
  const int my_key = j0t + n;
  const bool key_ok = my_key < len;
  KFrag<T, D> kf[HW], vf[HW];
  f32x4 dK[HW][D / 16], dV[HW][D / 16];
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    const int h = ws * HW + hl;
    if (h < H && key_ok) {
      kf[hl].load(kg + rx.off(h, my_key, D), g);
      vf[hl].load(vg + rx.off(h, my_key, D), g);
    } else {
      kf[hl].zero();
      vf[hl].zero();
    }
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) dK[hl][dt] = dV[hl][dt] = zero4();
  }
  // ---- pair-owner: own keys (lane % 16) x streamed rows [ws*RWS, +RWS) ----
  const int pk = lane & 15;
  const float4 pos_j = use_e ? ra.pos(ev.pos4, j0t + pk < len ? j0t + pk : (len > 0 ? len - 1 : 0))
                             : float4{0.f, 0.f, 0.f, 0.f};

  // PF (float32 with QOS): the next chunk's qt / dO rows and per-row scalars
  // are loaded into registers (from clamped rows) while this chunk runs and
  // written to LDS at the start of the next, instead of being loaded and
  // waited for there: cfg4 cols 19.72 -> 19.24 ms, B=256 L=768 H=12 D=32
  // C=16 8.49 -> 8.13 ms. Only where the LDS plan already allows one
  // workgroup per CU (over 80 KB): elsewhere the registers cost a workgroup
  // per CU (H = 8, D = 32, C = 16: 0.79 -> 1.07 ms; H = 4: 0.50 -> 0.58),
  // and not past HW D = 128 (spills).
  constexpr bool PF = Cfg::QOS && !BF && HW * D <= 128 && Cfg::LDS_BYTES > 80 * 1024;
  using V16 = typename VecOf<T>::type;
  constexpr int VEC = 16 / Cfg::ESZ;
  constexpr int PER_ROW = D / VEC;
  constexpr int QIT = PF ? (HP * KC * PER_ROW + NT - 1) / NT : 1;  // rows' 16-byte items per thread
  constexpr int LIT = PF ? (HP * KC + NT - 1) / NT : 1;            // per-row scalars per thread
  V16 qraw[QIT], oraw[QIT];
  float lraw[LIT][4];
  auto prefetch = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int it = 0; it < QIT; ++it) {
      const int idx = tid + it * NT;
      if (idx < H * KC * PER_ROW) {
        const int dv = idx % PER_ROW, il = (idx / PER_ROW) % KC, h = idx / (PER_ROW * KC);
        const int i = min(c + il, len - 1);
        qraw[it] = *reinterpret_cast<const V16*>(qg + rx.off(h, i, D) + dv * VEC);
        oraw[it] = *reinterpret_cast<const V16*>(dog + ra.off(h, i, D) + dv * VEC);
      }
    }
#pragma unroll
    for (int it = 0; it < LIT; ++it) {
      const int idx = tid + it * NT;
      if (idx < H * KC) {
        const int il = idx % KC, h = idx / KC;
        const long v = ra.vec(h, min(c + il, len - 1));
        lraw[it][0] = prm.lse[v];
        lraw[it][1] = prm.dsum[v];
        lraw[it][2] = (act && prm.bias) ? prm.dob[v] : 0.f;
        lraw[it][3] = prm.lse_z[v];
      }
    }
  };
  // (Padded events of length 0 get one workgroup, for their padding rows:
  // nothing is loaded for them.)
  if constexpr (PF)
    if (len > 0) prefetch(0);

  // ---- ER: this wave's streamed rows' u and w~ go to its blocks of the E
  // tile by direct loads, [row][u, w~][head][C + 4] (the pad slot of a head
  // repeats its last quad; heads past H and rows past the event are clamped,
  // feeding only outputs that are never used), and the rows' positions to
  // registers, a phase before they are used ----
  constexpr bool ER = Cfg::ER;
  unsigned char* ul = reinterpret_cast<unsigned char*>(Es) + ws * RWS * 2 * Cfg::UWL_SLOTS * 16;
  float4 pin[ER ? RWS : 1];
  const long uw_base = ra.off(0, 0, C);
  const unsigned uw_bytes = (unsigned)(((long)(H - 1) * ra.hs + (long)(len > 0 ? len - 1 : 0) * ra.ts + 1) * C * 4);
  const __amdgpu_buffer_rsrc_t urs = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(ug + uw_base), (short)0, (int)uw_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(wg_ + uw_base), (short)0, (int)uw_bytes, 0x00020000);
  auto issue_uw = [&](int c) __attribute__((always_inline)) {
    if constexpr (ER) {
      constexpr int SPH = Cfg::UWL_ROW / 16;  // slots per head
#pragma unroll
      for (int ri = 0; ri < RWS; ++ri) {
        const int i = min(c + ws * RWS + ri, len - 1);
        pin[ri] = ra.pos(ev.pos4, i);
#pragma unroll
        for (int t = 0; t < Cfg::UWL_LOADS; ++t) {
          const int sl = 64 * t + lane;
          const int h = min(sl / SPH, H - 1), q = min(sl % SPH, C / 4 - 1);
          const int voff = (int)(((long)h * ra.hs + (long)i * ra.ts) * C + 4 * q) * 4;
          if (sl < Cfg::UWL_SLOTS) {
            if (attn)
              __builtin_amdgcn_raw_ptr_buffer_load_lds(
                  urs, (__attribute__((address_space(3))) void*)(ul + ((2 * ri) * Cfg::UWL_SLOTS + 64 * t) * 16), 16, voff, 0, 0, 0);
            if (act)
              __builtin_amdgcn_raw_ptr_buffer_load_lds(
                  wrs, (__attribute__((address_space(3))) void*)(ul + ((2 * ri + 1) * Cfg::UWL_SLOTS + 64 * t) * 16), 16, voff, 0, 0, 0);
          }
        }
      }
    }
  };
  if constexpr (ER)
    if (use_e && len > 0) issue_uw(0);

  for (int c0 = 0; c0 < len; c0 += KC) {
    // ER: this chunk's u / w~ blocks (and, with PF, the prefetched rows)
    // have landed.
    if constexpr (ER) wait_vmem();
    if constexpr (PF) {
      // ---- PF: stage the prefetched rows (zero past the event), then load
      // the next chunk's ----
#pragma unroll
      for (int it = 0; it < QIT; ++it) {
        const int idx = tid + it * NT;
        if (idx < H * KC * PER_ROW) {
          const int dv = idx % PER_ROW, il = (idx / PER_ROW) % KC, h = idx / (PER_ROW * KC);
          const bool ok = c0 + il < len;
          V16 qv = VecOf<T>::zero(), ov = VecOf<T>::zero();
          if (ok) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) qv[e] = (T)((float)qraw[it][e] * prm.scale);
            ov = oraw[it];
          }
          *reinterpret_cast<V16*>(Qs + (h * KC + il) * Cfg::QO_ROW + dv * VEC) = qv;
          *reinterpret_cast<V16*>(Os + (h * KC + il) * Cfg::QO_ROW + dv * VEC) = ov;
        }
      }
#pragma unroll
      for (int it = 0; it < LIT; ++it) {
        const int idx = tid + it * NT;
        if (idx < H * KC) {
          const bool ok = c0 + idx % KC < len;
          Lv[idx] = ok ? lraw[it][0] * kLog2e : 0.f;
          Lv[HP * KC + idx] = ok ? lraw[it][1] : 0.f;
          Lv[2 * HP * KC + idx] = ok ? lraw[it][2] : 0.f;
          Lv[3 * HP * KC + idx] = ok ? lraw[it][3] : 0.f;
        }
      }
      if (c0 + KC < len) prefetch(c0 + KC);
    }
    // ---- stage the chunk's streamed rows: qt, dO (QOS), lse2, D, dob ----
    if constexpr (Cfg::QOS && !PF) {
      using V16 = typename VecOf<T>::type;
      constexpr int VEC = 16 / Cfg::ESZ;
      constexpr int PER_ROW = D / VEC;
      const int total = H * KC * PER_ROW;
      for (int idx = tid; idx < total; idx += NT) {
        const int dv = idx % PER_ROW;
        const int il = (idx / PER_ROW) % KC;
        const int h = idx / (PER_ROW * KC);
        const int i = c0 + il;
        V16 qv = VecOf<T>::zero(), ov = VecOf<T>::zero();
        if (i < len) {
          const V16 raw = *reinterpret_cast<const V16*>(qg + rx.off(h, i, D) + dv * VEC);
#pragma unroll
          for (int e = 0; e < VEC; ++e) qv[e] = (T)((float)raw[e] * prm.scale);
          ov = *reinterpret_cast<const V16*>(dog + ra.off(h, i, D) + dv * VEC);
        }
        *reinterpret_cast<V16*>(Qs + (h * KC + il) * Cfg::QO_ROW + dv * VEC) = qv;
        *reinterpret_cast<V16*>(Os + (h * KC + il) * Cfg::QO_ROW + dv * VEC) = ov;
      }
    }
    for (int idx = tid; !PF && idx < H * KC; idx += NT) {
      const int il = idx % KC, h = idx / KC;
      const int i = c0 + il;
      const bool ok = i < len;
      Lv[idx] = ok ? prm.lse[ra.vec(h, i)] * kLog2e : 0.f;
      Lv[HP * KC + idx] = ok ? prm.dsum[ra.vec(h, i)] : 0.f;
      Lv[2 * HP * KC + idx] = (ok && act && prm.bias) ? prm.dob[ra.vec(h, i)] : 0.f;
      Lv[3 * HP * KC + idx] = ok ? prm.lse_z[ra.vec(h, i)] : 0.f;
    }
    // ---- pair-owner: E of (streamed rows, own keys), u.E and w~.E ----
    if constexpr (ER) {
      if (use_e) {
        const int hn = n < HP ? n : HP - 1;
#pragma unroll
        for (int ri = 0; ri < RWS; ++ri) {
          const int il = ws * RWS + ri;
          const CFrag<T, C> ef = embed_cfrag<C>(pin[ri], pos_j, prm.freq, g);  // B = E_i[c, j]: lane n = key
#pragma unroll
          for (int op = 0; op < 2; ++op) {
            if (!(op == 0 ? attn : act)) continue;
            CFrag<T, C> af;  // A = u_i[h, c] (w~_i): lane n = head
            const unsigned char* blk = ul + (2 * ri + op) * Cfg::UWL_SLOTS * 16 + hn * Cfg::UWL_ROW;
#pragma unroll
            for (int ct = 0; ct < C / 16; ++ct) af.v[ct] = *reinterpret_cast<const f32x4*>(blk + (16 * ct + 4 * g) * 4);
            const f32x4 ue = mma_c<C>(af, ef, zero4());  // [h = 4g + r][j = n]
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (4 * g + r < H) UWs[op * HP * 16 * UWR + ((4 * g + r) * 16 + n) * UWR + il] = ue[r];
          }
        }
        // The blocks are read: the next chunk's rows may overwrite them.
        if (c0 + KC < len) {
          wave_lds_sync();
          issue_uw(c0 + KC);
        }
      }
    } else if (use_e) {
      using EL = typename Cfg::EL;  // lane slot el -> key el & 15, rows (el >> 4) + 4 k4
      const int el = EL::slot(lane), epart = EL::part(lane);
#pragma unroll
      for (int k4 = 0; k4 < EL::EPL; ++k4) {
        const int il = ws * RWS + (el >> 4) + 4 * k4;
        const int i = c0 + il;
        const float4 pi = ra.pos(ev.pos4, i < len ? i : len - 1);
        write_embedding<T, C, EL::SPLIT>(Es + (il * 16 + pk) * Cfg::E_ROW, pi, pos_j, prm.freq, epart);
      }
      wave_lds_sync();
#pragma unroll
      for (int ri = 0; ri < RWS; ++ri) {
        const int il = ws * RWS + ri;
        const int i = c0 + il;
        const bool ok = i < len && n < H;
        CFrag<T, C> ef;  // B = E_i[c, j]: lane n = key
        ef.load(Es + (il * 16 + n) * Cfg::E_ROW, g);
        if (attn) {
          CFrag<T, C> uf;  // A = u_i[h, c]: lane n = head
          if (ok)
            uf.load(ug + ra.off(n, i, C), g);
          else
            uf.zero();
          const f32x4 ue = mma_c<C>(uf, ef, zero4());  // [h = 4g + r][j = n]
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (4 * g + r < H) UWs[((4 * g + r) * 16 + n) * UWR + il] = ue[r];
        }
        if (act) {
          CFrag<T, C> wf;
          if (ok)
            wf.load(wg_ + ra.off(n, i, C), g);
          else
            wf.zero();
          const f32x4 we = mma_c<C>(wf, ef, zero4());
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (4 * g + r < H) UWs[HP * 16 * UWR + ((4 * g + r) * 16 + n) * UWR + il] = we[r];
        }
      }
    }
    __syncthreads();

    // ---- head-owner: S = qt k^T + u.E, P, dP, dS; dv += dO^T P, dk += qt^T dS ----
#pragma unroll
    for (int hl = 0; hl < HW; ++hl) {
      const int h = ws * HW + hl;
      if (h >= H) continue;
      f32x4 S[NS], dP[NS], dS[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const float* us = UWs + (h * 16 + n) * UWR + 16 * s + 4 * g;
        const f32x4 ue = attn ? *reinterpret_cast<const f32x4*>(us) : zero4();
        const f32x4 we = act ? *reinterpret_cast<const f32x4*>(us + HP * 16 * UWR) : zero4();
        KFrag<T, D> qa, oa;  // A = qt_i[d], dO_i[d]: lane n = streamed row 16s + n
        if constexpr (Cfg::QOS) {
          qa.load(Qs + (h * KC + 16 * s + n) * Cfg::QO_ROW, g);
          oa.load(Os + (h * KC + 16 * s + n) * Cfg::QO_ROW, g);
        } else {
          int i = c0 + 16 * s + n;
          i = i < len ? i : len - 1;
          qa.load_scaled(qg + rx.off(h, i, D), g, prm.scale);
          oa.load(dog + ra.off(h, i, D), g);
        }
        S[s] = mma_k<D>(qa, kf[hl], ue);
        dP[s] = mma_k<D>(oa, vf[hl], we);
        unsigned vm = 0;
        f32x4 lse4, d4, dob4, z4;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int il = 16 * s + 4 * g + r;
          vm |= ((c0 + il < len && key_ok) ? 1u : 0u) << r;
          lse4[r] = Lv[h * KC + il];
          d4[r] = Lv[HP * KC + h * KC + il];
          dob4[r] = Lv[2 * HP * KC + h * KC + il];
          z4[r] = Lv[3 * HP * KC + h * KC + il];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool ok = (vm >> r) & 1u;
          // P / Z, as the rows kernel's accumulators hold it.
          const float p = exp2f_fast(__builtin_fmaf(S[s][r], kLog2e, -lse4[r]) - z4[r]);
          S[s][r] = ok ? p : 0.f;
          dP[s][r] = dP[s][r] + dob4[r];
          dS[s][r] = S[s][r] * (dP[s][r] - d4[r]);
        }
      }
      JFrag<T, NS> pf, dsf;
      pf.from_tiles(S);
      dsf.from_tiles(dS);
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        JFrag<T, NS> ot, qt;
        if constexpr (Cfg::QOS) {
          ot.load_tr(Os + h * KC * Cfg::QO_ROW, Cfg::QO_ROW, 16 * dt, g, n);
          qt.load_tr(Qs + h * KC * Cfg::QO_ROW, Cfg::QO_ROW, 16 * dt, g, n);
        } else {
#pragma unroll
          for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int i = c0 + 16 * s + 4 * g + r;
              const bool ok = i < len;
              const int ic = ok ? i : 0;
              ot.v[4 * s + r] = ok ? (float)dog[ra.off(h, ic, D) + 16 * dt + n] : 0.f;
              qt.v[4 * s + r] = ok ? (float)qg[rx.off(h, ic, D) + 16 * dt + n] * prm.scale : 0.f;
            }
        }
        dV[hl][dt] = mma_j(ot, pf, dV[hl][dt]);
        dK[hl][dt] = mma_j(qt, dsf, dK[hl][dt]);
      }
    }
    __syncthreads();
  }

  T* dkg = reinterpret_cast<T*>(prm.dk);
  T* dvg = reinterpret_cast<T*>(prm.dv);
#pragma unroll
  for (int hl = 0; hl < HW; ++hl) {
    const int h = ws * HW + hl;
    if (h >= H || !key_ok) continue;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
      store4<T>(dkg + rx.off(h, my_key, D) + 16 * dt + 4 * g, dK[hl][dt]);
      store4<T>(dvg + rx.off(h, my_key, D) + 16 * dt + 4 * g, dV[hl][dt]);
    }
  }
  zero_pad_rows<T>(ev, eb, rx, rx, key0, Cfg::KEYS, D, tid, NT, dkg, nullptr, 1);
  zero_pad_rows<T>(ev, eb, rx, rx, key0, Cfg::KEYS, D, tid, NT, dvg, nullptr, 1);
}

// ---------------------------------------------------------------------------
// Dispatch.
// ---------------------------------------------------------------------------
// The static choice of each kernel is the split with the most waves per
// 16-row tile that fits LDS, with 16-key (row) chunks first (measured on
// gfx950: 18.4 against 19.1 ms for the float32 backward at B=256, L=768,
// H=12, D=32, C=16, and 3.9 against 6.7 ms at H=4, D=C=16); the plan bits
// FST_PLAN_BWD_T16 / T32 / T64 fix the rows (rows kernel) and keys (cols
// kernel) per workgroup, FST_PLAN_BWD_KC16 / KC32 the keys (rows kernel) and
// rows (cols kernel) per chunk, each kernel taking the first fitting value
// of a group left empty.
template <template <typename, int, int, int, int, int> class Cfg, typename T, int HP, int D, int C>
struct BwdPick {
  template <int NW, int NS>
  using F = Cfg<T, HP, D, C, NW, NS>;
  static constexpr int STATIC = pick_split<F>(0, 0, 1);
  static constexpr int NW = STATIC ? STATIC / 10 : 4, NS = STATIC ? STATIC % 10 : 1;
  using Sel = F<NW, NS>;
  static constexpr bool OK = STATIC != 0;
};

// Passes of the rows kernel's static choice: one where the lane state of
// the one-pass form stays small ((HP / NW) D + (16 / NW) C <= 256: Q, dO,
// dQ and sum P k per head, u, w~, H and G per row; at B=256 L=768 H=12
// D=32 C=16 in float32 one pass took 7.06 against 9.72 ms), two where it
// would spill heavily (cfg4, D = C = 64, four waves: 82.8 against 41.2 ms).
// Eight waves halve the state: at cfg4 one pass (51 registers spilled)
// took 22.7 ms against 31.7 for two.
template <int HP, int D, int C, int NW>
constexpr int rows_static_passes() {
  return (HP / NW) * D + (16 / NW) * C <= 256 ? 1 : 2;
}

template <typename T, int HP, int D, int C, int NW, int NS>
int bwd_launch_v(const BwdParams& prm, int which, hipStream_t stream, int grid, bool query, int* rows) {
  using R = BwdRowsCfg<T, HP, D, C, NW, NS>;
  using K = BwdColsCfg<T, HP, D, C, NW, NS>;
  if (which == 0) {
    if constexpr (!R::FITS) {
      return FST_EUNSUPPORTED;
    } else {
      *rows = R::ROWS;
      if (query) return FST_OK;
      const int passes = (prm.flags & FST_PLAN_BWD_PASS1)   ? 1
                         : (prm.flags & FST_PLAN_BWD_PASS2) ? 2
                                                            : rows_static_passes<HP, D, C, NW>();
      auto kern = passes == 1 ? bwd_rows_kernel<T, HP, D, C, NW, NS, 1> : bwd_rows_kernel<T, HP, D, C, NW, NS, 2>;
      if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, R::LDS_BYTES) !=
          hipSuccess)
        return FST_ELAUNCH;
      if (grid > 0) hipLaunchKernelGGL(kern, dim3(grid), dim3(R::THREADS), R::LDS_BYTES, stream, prm);
      return hipGetLastError() == hipSuccess ? FST_OK : FST_ELAUNCH;
    }
  }
  if constexpr (!K::FITS) {
    return FST_EUNSUPPORTED;
  } else {
    *rows = K::KEYS;
    if (query) return FST_OK;
    auto kern = bwd_cols_kernel<T, HP, D, C, NW, NS>;
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, K::LDS_BYTES) !=
        hipSuccess)
      return FST_ELAUNCH;
    if (grid > 0) hipLaunchKernelGGL(kern, dim3(grid), dim3(K::THREADS), K::LDS_BYTES, stream, prm);
    return hipGetLastError() == hipSuccess ? FST_OK : FST_ELAUNCH;
  }
}

// The FST_PLAN_BWD_* bits offered: a value of a group is offered when both
// kernels have a fitting split with it.
template <typename T, int HP, int D, int C>
constexpr int bwd_split_plans() {
  using PR = BwdPick<BwdRowsCfg, T, HP, D, C>;
  using PC = BwdPick<BwdColsCfg, T, HP, D, C>;
  return (split_plans<PR::template F>(FST_PLAN_BWD_T16, FST_PLAN_BWD_KC16, FST_PLAN_BWD_W8) &
          split_plans<PC::template F>(FST_PLAN_BWD_T16, FST_PLAN_BWD_KC16, FST_PLAN_BWD_W8)) |
         FST_PLAN_BWD_PASS1 | FST_PLAN_BWD_PASS2;
}

// Launches (or, with query, only checks) the rows (which = 0) or cols
// kernel's split that the plan bits of prm.flags name; *rows receives its
// rows (keys) per workgroup.
template <typename T, int HP, int D, int C>
int bwd_launch_t(const BwdParams& prm, int which, hipStream_t stream, int grid, bool query, int* rows) {
  using PR = BwdPick<BwdRowsCfg, T, HP, D, C>;
  using PC = BwdPick<BwdColsCfg, T, HP, D, C>;
  *rows = 0;
  if constexpr (!PR::OK || !PC::OK) {
    return FST_EUNSUPPORTED;
  } else {
    const int nw = plan_nw(prm.flags, bit_index(FST_PLAN_BWD_T16), bit_index(FST_PLAN_BWD_W8));
    const int ns = plan_ns(prm.flags, bit_index(FST_PLAN_BWD_KC16));
    const int split = which == 0 ? pick_split<PR::template F>(nw, ns, 1) : pick_split<PC::template F>(nw, ns, 1);
    switch (split) {
      case 11: return bwd_launch_v<T, HP, D, C, 1, 1>(prm, which, stream, grid, query, rows);
      case 12: return bwd_launch_v<T, HP, D, C, 1, 2>(prm, which, stream, grid, query, rows);
      case 21: return bwd_launch_v<T, HP, D, C, 2, 1>(prm, which, stream, grid, query, rows);
      case 22: return bwd_launch_v<T, HP, D, C, 2, 2>(prm, which, stream, grid, query, rows);
      case 41: return bwd_launch_v<T, HP, D, C, 4, 1>(prm, which, stream, grid, query, rows);
      case 42: return bwd_launch_v<T, HP, D, C, 4, 2>(prm, which, stream, grid, query, rows);
      case 81: return bwd_launch_v<T, HP, D, C, 8, 1>(prm, which, stream, grid, query, rows);
      case 82: return bwd_launch_v<T, HP, D, C, 8, 2>(prm, which, stream, grid, query, rows);
      default: return FST_EUNSUPPORTED;
    }
  }
}

}  // namespace fst
