// C ABI of the flash-spacetime library (declared in include/flash_spacetime.h):
// argument validation, the frequency table, the per-event work list and the
// kernel launches. Nothing here allocates, frees or synchronises; all work
// goes onto the caller's stream.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "fst_kernels.h"

namespace fst {

static thread_local char g_last_error[512] = "";

static int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
static int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

static size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

static bool supported_dim(int x) { return x == 16 || x == 32 || x == 48 || x == 64; }

static int head_padding(int H) { return H <= 4 ? 4 : (H <= 8 ? 8 : (H <= 12 ? 12 : 16)); }

// Head padding of the bf16 rows kernel: where its four-wave instance would
// spill, heads are padded to the next multiple of 8 so that it runs eight
// waves (padded heads compute on a real head's data and store nothing). The
// cols kernel keeps head_padding: the scratch between them is laid out by H.
// The eight-wave, one-workgroup plan (FST_PLAN_ROWS_W8) pads to a multiple
// of 8 likewise; the four-wave plan and the eight-wave, two-workgroup plan
// (which gives waves 4 to 7 one head fewer where 8 does not divide the
// padding) keep head_padding.
static int rows_head_padding(int dtype, int flags, int H, int D, int C) {
  const int hp = head_padding(H);
  if (dtype != FST_BF16) return hp;
  if (flags & FST_PLAN_ROWS_W8) return (hp + 7) & ~7;
  if (flags & (FST_PLAN_ROWS_W4 | FST_PLAN_ROWS_W8X2)) return hp;
  if (hp % 8 != 0 && rows_wave_load(hp, D, C) >= 160) return hp + 4;
  return hp;
}

// fp32 frequency ladder exp(-i * ln(1e4) / (C/2)) evaluated with the same
// fp32 steps as the reference (reference.py:45-56): fp32 log of 1e4, fp32
// division by C/2, fp32 product with i, exponential rounded to fp32.
static void frequencies(int C, float* out) {
  const float half = (float)C / 2.0f;
  const float lg = (float)std::log(10000.0);
  const float step = -(lg / half);
  for (int i = 0; i < C / 2; ++i) {
    const float arg = (float)i * step;
    out[i] = (float)std::exp((double)arg);
  }
}

static void freq_table(int C, FreqTable& ft) {
  std::memset(&ft, 0, sizeof(ft));
  float f[32];
  frequencies(C, f);
  const double inv2pi = 0.15915494309189533576888376337251;
  for (int i = 0; i < C / 2; ++i) {
    const double gd = (double)f[i] * inv2pi;
    ft.ghi[i] = (float)gd;
    ft.glo[i] = (float)(gd - (double)ft.ghi[i]);
    // |x| <= 4096; v_sin_f32 / v_cos_f32 accept +-256 revolutions.
    if (4096.0 * gd > 255.0) ft.reduce_mask |= 1u << i;
  }
}

// Inclusive scan of x over the work list's 1024 threads under op (a sum or a
// max; 0 is the identity for the values scanned here): within each wave by
// lane shuffles, then each thread combines the totals of the waves before it
// (broadcast LDS reads after one barrier). total receives the workgroup's
// result. wsum (16 ints) is reused: the caller puts a barrier between calls.
template <typename Op>
__device__ int block_scan(int x, int* wsum, int& total, Op op) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(x, off);
    if (lane >= off) x = op(x, o);
  }
  if (lane == 63) wsum[wv] = x;
  __syncthreads();
  int pre = 0;
  total = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int s = wsum[k];
    if (k < wv) pre = op(pre, s);
    total = op(total, s);
  }
  return op(pre, x);
}

// Exclusive prefix sums of val(i), i < n, into out[0 .. n] (out[0] = 0);
// one workgroup, chunks of 1024 with a carry.
template <typename F>
__device__ void scan_steps(int n, F val, int32_t* out, int* wsum) {
  const int t = threadIdx.x;
  if (t == 0) out[0] = 0;
  int carry = 0;
  for (int base = 0; base < n; base += 1024) {
    const int i = base + t;
    int total;
    const int inc = block_scan(i < n ? val(i) : 0, wsum, total, [](int a, int c) { return a + c; });
    if (i < n) out[i + 1] = carry + inc;
    carry += total;
    __syncthreads();
  }
}

// Number of row blocks of each event and their prefix sum, over the events
// in index order, or in the order perm gives when not null; one workgroup.
// Padded events always get one block so that their padding rows are zeroed.
__device__ void blkcum_steps(const EventSpec& ev, int rows, const int32_t* perm, int32_t* blkcum, int* wsum) {
  scan_steps(
      ev.B,
      [&](int b) {
        int tok0, len;
        event_range(ev, perm ? perm[b] : b, tok0, len);
        return len > 0 ? (len + rows - 1) / rows : (ev.packed ? 0 : 1);
      },
      blkcum, wsum);
}

// Schedule of the tile kernels: the events ordered by decreasing valid
// length (ties by index; lengths past 2^18 - 1 count as 2^18 - 1), one
// workgroup. Up to 1024 events each thread ranks one key by counting the
// larger ones (the keys are distinct, so the ranks are a permutation; one
// barrier, broadcast LDS reads); up to 8192 a bitonic sort with the keys in
// registers (bitonic_regs). Past 8192 events the identity order is used.
constexpr int kSortMax = 8192;
constexpr int kRankMax = 1024;

__device__ int sort_key(const EventSpec& ev, int i) {
  if (i >= ev.B) return -1;
  int tok0, l;
  event_range(ev, i, tok0, l);
  l = l < (1 << 18) - 1 ? l : (1 << 18) - 1;
  return (l << 13) | (kSortMax - 1 - i);
}

// One compare-exchange step at distance J < KPT: both keys of each pair are
// in the thread's registers. Position p = KPT t + r; the pair's lower
// position keeps the larger key where bit k of p is clear (a descending
// block), the smaller one elsewhere.
template <int KPT, int J>
__device__ __forceinline__ void bitonic_in_thread(int* x, int k) {
  if constexpr (J < KPT) {
#pragma unroll
    for (int r = 0; r < KPT; ++r)
      if ((r & J) == 0) {
        const int a = x[r], b = x[r | J];
        const bool desc = ((KPT * (int)threadIdx.x + r) & k) == 0;
        x[r] = desc ? max(a, b) : min(a, b);
        x[r | J] = desc ? min(a, b) : max(a, b);
      }
  }
}

// Bitonic sort, descending, of the 1024 KPT keys thread t holds at
// positions KPT t .. KPT t + KPT - 1 (registers x). Steps whose pairs lie in
// one thread (distance j < KPT) or one wave (j < 64 KPT: lane shuffles) take
// no barrier; the others (j >= 64 KPT) exchange through LDS, two barriers
// each.
template <int KPT>
__device__ void bitonic_regs(int* x, int* keys) {
  const int t = threadIdx.x;
  for (int k = 2; k <= 1024 * KPT; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j < KPT) {
        if (j == 1)
          bitonic_in_thread<KPT, 1>(x, k);
        else if (j == 2)
          bitonic_in_thread<KPT, 2>(x, k);
        else
          bitonic_in_thread<KPT, 4>(x, k);
      } else if (j < 64 * KPT) {
#pragma unroll
        for (int r = 0; r < KPT; ++r) {
          const int p = KPT * t + r;
          const int o = __shfl_xor(x[r], j / KPT);
          const bool keep_max = ((p & j) == 0) == ((p & k) == 0);
          x[r] = keep_max ? max(x[r], o) : min(x[r], o);
        }
      } else {
#pragma unroll
        for (int r = 0; r < KPT; ++r) keys[KPT * t + r] = x[r];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < KPT; ++r) {
          const int p = KPT * t + r;
          const int o = keys[p ^ j];
          const bool keep_max = ((p & j) == 0) == ((p & k) == 0);
          x[r] = keep_max ? max(x[r], o) : min(x[r], o);
        }
        __syncthreads();
      }
    }
}

template <int KPT>
__device__ void sort_regs(const EventSpec& ev, int32_t* perm, int* keys) {
  const int t = threadIdx.x;
  int x[KPT];
#pragma unroll
  for (int r = 0; r < KPT; ++r) x[r] = sort_key(ev, KPT * t + r);
  bitonic_regs<KPT>(x, keys);
#pragma unroll
  for (int r = 0; r < KPT; ++r)
    if (KPT * t + r < ev.B) perm[KPT * t + r] = kSortMax - 1 - (x[r] & (kSortMax - 1));
}

__device__ void sort_steps(const EventSpec& ev, int32_t* perm, int* keys) {
  const int t = threadIdx.x, B = ev.B;
  if (B > kSortMax) {
    for (int i = t; i < B; i += 1024) perm[i] = i;
    return;
  }
  if (B <= kRankMax) {
    if (t < B) keys[t] = sort_key(ev, t);
    __syncthreads();
    if (t < B) {
      const int mine = keys[t];
      int rank = 0;
      for (int j = 0; j < B; ++j) rank += keys[j] > mine;
      perm[rank] = kSortMax - 1 - (mine & (kSortMax - 1));
    }
    return;
  }
  if (B <= 2048)
    sort_regs<2>(ev, perm, keys);
  else if (B <= 4096)
    sort_regs<4>(ev, perm, keys);
  else
    sort_regs<8>(ev, perm, keys);
}

// Packed offsets as the kernels read them: cus[b] = the running maximum of
// cu[0 .. b], clamped to [0, T], so events never overlap, never leave the
// tensor and their row blocks never outnumber the per-tile slots the
// workspace sizes from T (ceil(T / rows) + B). *status = 1 when the caller's
// offsets were malformed (cu[0] != 0, a decrease, or cu[B] > T); the tile
// kernels then write NaN into every event's rows instead of computing.
// cu[B] < T is allowed: tokens past cu[B] belong to no event and are left
// unwritten.
__device__ void sanitize_steps(const int32_t* cu, int B, int T, int32_t* cus, int32_t* status, int* wsum) {
  const int t = threadIdx.x;
  int bad = 0, carry = 0;
  for (int base = 0; base <= B; base += 1024) {
    const int b = base + t;
    int x = 0;
    if (b <= B) {
      x = cu[b];
      if (b == 0 ? x != 0 : x < cu[b - 1]) bad = 1;
      if (b == B && x > T) bad = 1;
    }
    int total;
    const int inc = block_scan(x, wsum, total, [](int a, int c) { return max(a, c); });
    if (b <= B) cus[b] = min(max(carry, inc), T);
    carry = max(carry, total);
    __syncthreads();
  }
  bad = __syncthreads_or(bad);
  if (t == 0) *status = bad;
}

// The padding-last schedule's prefix sums (EventSpec::vp): valid 16-row tiles
// of the padded events in XCD order, entry x S + j for XCD x's j-th event
// (rank 8 j + (j odd ? 7 - x : x), as tile_block deals them), 0 past the
// events; an empty event keeps one tile (its zero dW / db slot).
__device__ void valid_tiles_steps(const EventSpec& ev, const int32_t* perm, int32_t* vp, int* wsum) {
  const int B = ev.B, S = (B + 7) >> 3;
  scan_steps(
      8 * S,
      [&](int idx) {
        const int x = idx / S, j = idx - x * S, r = 8 * j + ((j & 1) ? 7 - x : x);
        if (r >= B) return 0;
        int tok0, len;
        event_range(ev, perm[r], tok0, len);
        return len > 0 ? (len + 15) >> 4 : 1;
      },
      vp, wsum);
}

// The work list of one operator call in one launch (one workgroup, steps
// separated by barriers, which also order the global writes of perm before
// their reads): for packed events the sanitised offsets and the call status
// (sanitize_steps; padded calls get status 0); row-block prefix sums in
// event order for the row-block sizes rows_a and, when blk_b is not null,
// rows_b; the length-sorted order perm; for packed events the prefix sums in
// perm order (scum_a, scum_b), which are the tile kernels' schedule.
__global__ __launch_bounds__(1024) void worklist_kernel(const int32_t* lens, int packed, int B, int L, int T,
                                                        int rows_a, int32_t* blk_a, int rows_b, int32_t* blk_b,
                                                        int32_t* perm, int32_t* scum_a, int32_t* scum_b,
                                                        int32_t* cus, int32_t* status, int32_t* vp) {
  extern __shared__ int keys[];
  __shared__ int wsum[16];
  if (packed) {
    sanitize_steps(lens, B, T, cus, status, wsum);
  } else if (threadIdx.x == 0) {
    *status = 0;
  }
  __syncthreads();
  EventSpec ev;
  ev.lens = packed ? cus : lens;
  ev.packed = packed;
  ev.B = B;
  ev.L = L;
  ev.T = T;
  blkcum_steps(ev, rows_a, nullptr, blk_a, wsum);
  // The second family's lists equal the first's when its blocks are as tall
  // (the bf16 backward: 16 rows and 16 keys): copied instead of rescanned.
  const bool same = rows_b == rows_a;
  if (blk_b && !same) blkcum_steps(ev, rows_b, nullptr, blk_b, wsum);
  sort_steps(ev, perm, keys);
  __syncthreads();
  if (scum_a) blkcum_steps(ev, rows_a, perm, scum_a, wsum);
  if (scum_b && !same) blkcum_steps(ev, rows_b, perm, scum_b, wsum);
  if (same) {
    for (int i = threadIdx.x; i <= B; i += blockDim.x) {
      if (blk_b) blk_b[i] = blk_a[i];
      if (scum_b) scum_b[i] = scum_a[i];
    }
  }
  if (vp && !packed) valid_tiles_steps(ev, perm, vp, wsum);
}

static int launch_worklist(const int32_t* lens, bool packed, int B, int L, int T, int rows_a, int32_t* blk_a,
                           int rows_b, int32_t* blk_b, int32_t* perm, int32_t* scum_a, int32_t* scum_b,
                           int32_t* cus, int32_t* status, hipStream_t st, int32_t* vp = nullptr) {
  int p2 = 1;
  while (p2 < B && p2 < kSortMax) p2 <<= 1;
  const int lds = B > kSortMax ? 0 : p2 * (int)sizeof(int);
  if (hipFuncSetAttribute((const void*)worklist_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                          kSortMax * (int)sizeof(int)) != hipSuccess)
    return FST_ELAUNCH;
  hipLaunchKernelGGL(worklist_kernel, dim3(1), dim3(1024), lds, st, lens, packed ? 1 : 0, B, L, T, rows_a, blk_a,
                     rows_b, blk_b, perm, packed ? scum_a : nullptr, packed ? scum_b : nullptr, cus, status,
                     packed ? nullptr : vp);
  return hipGetLastError() == hipSuccess ? FST_OK : FST_ELAUNCH;
}

typedef int (*fwd_dispatch_fn)(const FwdParams&, int, int, hipStream_t, int, bool, int*);

static fwd_dispatch_fn fwd_table(int dtype, int D) {
  if (dtype == FST_BF16) {
    switch (D) {
      case 16: return fwd_dispatch_bf16_16;
      case 32: return fwd_dispatch_bf16_32;
      case 48: return fwd_dispatch_bf16_48;
      case 64: return fwd_dispatch_bf16_64;
    }
  } else if (dtype == FST_F32) {
    switch (D) {
      case 16: return fwd_dispatch_f32_16;
      case 32: return fwd_dispatch_f32_32;
      case 48: return fwd_dispatch_f32_48;
      case 64: return fwd_dispatch_f32_64;
    }
  }
  return nullptr;
}

typedef int (*plans_fn)(int, int);

static int shape_plans(int dtype, int H, int D, int C) {
  plans_fn f = nullptr, b = nullptr;
  if (dtype == FST_BF16) {
    switch (D) {
      case 16: f = fwd_plans_bf16_16; b = bwd_plans_bf16_16; break;
      case 32: f = fwd_plans_bf16_32; b = bwd_plans_bf16_32; break;
      case 48: f = fwd_plans_bf16_48; b = bwd_plans_bf16_48; break;
      case 64: f = fwd_plans_bf16_64; b = bwd_plans_bf16_64; break;
    }
  } else if (dtype == FST_F32) {
    switch (D) {
      case 16: f = fwd_plans_f32_16; b = bwd_plans_f32_16; break;
      case 32: f = fwd_plans_f32_32; b = bwd_plans_f32_32; break;
      case 48: f = fwd_plans_f32_48; b = bwd_plans_f32_48; break;
      case 64: f = fwd_plans_f32_64; b = bwd_plans_f32_64; break;
    }
  }
  if (!f || H < 1 || H > 16) return 0;
  return f(head_padding(H), C) | b(head_padding(H), C);
}

// Longest event whose rows of all heads the bf16 kernels can address with
// 32-bit byte offsets: q, k, v rows (times 3 interleaved) and the u / w~
// scratch of the cols kernel (C values per row and head) must span less than
// 2^31 bytes. The same bound is kept for float32.
static int max_event_len(int dtype, int flags, int H, int D, int C) {
  const long long es = dtype == FST_BF16 ? 2 : 4;
  const long long xd = (long long)D * ((flags & FST_QKV_INTERLEAVED) ? 3 : 1);
  const long long span = (long long)H * es * (xd > C ? xd : C);
  const long long m = ((1LL << 31) - 1) / span;
  return m > 0x7fffffffLL ? 0x7fffffff : (int)m;
}

// The plan-bit groups of include/flash_spacetime.h: at most one bit each.
static const int kPlanGroups[] = {
    FST_PLAN_FWD_OCC2 | FST_PLAN_FWD_OCC3,
    FST_PLAN_ROWS_W4 | FST_PLAN_ROWS_W8 | FST_PLAN_ROWS_W8X2,
    FST_PLAN_COLS_OCC2 | FST_PLAN_COLS_OCC3,
    FST_PLAN_ROWS_KV_REG | FST_PLAN_ROWS_KV_LDS,
    FST_PLAN_FWD_KC16 | FST_PLAN_FWD_KC32,
    FST_PLAN_FWD_T16 | FST_PLAN_FWD_T32 | FST_PLAN_FWD_T64 | FST_PLAN_FWD_W8,
    FST_PLAN_BWD_T16 | FST_PLAN_BWD_T32 | FST_PLAN_BWD_T64 | FST_PLAN_BWD_W8,
    FST_PLAN_BWD_KC16 | FST_PLAN_BWD_KC32,
    FST_PLAN_BWD_PASS1 | FST_PLAN_BWD_PASS2,
};

static int check_common(int dtype, int flags, int B, int H, int L, int T, int D, int C) {
  if (dtype != FST_BF16 && dtype != FST_F32) return fail(FST_EINVAL, "dtype must be FST_BF16 or FST_F32, got %d", dtype);
  if (flags & ~(FST_ATTN_BIAS | FST_ACT_BIAS | FST_PACKED | FST_TOKEN_MAJOR | FST_QKV_INTERLEAVED | FST_PLAN_MASK))
    return fail(FST_EINVAL, "unknown flag bits 0x%x", flags);
  for (int group : kPlanGroups)
    if ((flags & group) & ((flags & group) - 1))
      return fail(FST_EINVAL, "plan bits 0x%x name two variants of one kernel knob", flags & group);
  if ((flags & FST_QKV_INTERLEAVED) && !(flags & (FST_PACKED | FST_TOKEN_MAJOR)))
    return fail(FST_EINVAL, "FST_QKV_INTERLEAVED needs a token-major layout (FST_PACKED or FST_TOKEN_MAJOR)");
  if ((flags & FST_PACKED) && (flags & FST_TOKEN_MAJOR))
    return fail(FST_EINVAL, "FST_TOKEN_MAJOR applies to the padded layout (packed is token-major already)");
  if (B < 0 || L < 0 || T < 0) return fail(FST_EINVAL, "negative size (B=%d, L=%d, T=%d)", B, L, T);
  if (H < 1 || H > 16) return fail(FST_EUNSUPPORTED, "heads must be in [1, 16], got %d", H);
  if (!supported_dim(D)) return fail(FST_EUNSUPPORTED, "head_dim D must be one of 16, 32, 48, 64, got %d", D);
  if (!supported_dim(C)) return fail(FST_EUNSUPPORTED, "channel count C must be one of 16, 32, 48, 64, got %d", C);
  // The kernels address one event's rows with 32-bit byte offsets (buffer
  // loads over the event's span): a padded event's rows of every head must
  // span less than 2 GiB. Packed events are bounded by the caller (the
  // lengths live on the device).
  if (!(flags & FST_PACKED) && L > max_event_len(dtype, flags, H, D, C))
    return fail(FST_EUNSUPPORTED, "padded events of %d tokens span 2^31 bytes or more (the kernels address at most %d "
                "tokens of this layout)", L, max_event_len(dtype, flags, H, D, C));
  const int plan = flags & FST_PLAN_MASK;
  if (plan & ~shape_plans(dtype, H, D, C))
    return fail(FST_EUNSUPPORTED, "plan bits 0x%x are not compiled for dtype %d, H=%d, D=%d, C=%d", plan, dtype, H, D,
                C);
  return FST_OK;
}

// Work list of one kernel family: blkcum [B+1] (row blocks in event order:
// the slots of per-tile outputs), perm [B] (events by decreasing length),
// scum [B+1] (packed: row blocks in perm order, the schedule), cus [B+1]
// (packed: the sanitised offsets the kernels read), status [1].
struct WorkList {
  int32_t *blkcum, *perm, *scum, *cus, *status;
};
static size_t blkcum_bytes(int B) { return align_up((size_t)(4 * B + 4) * sizeof(int32_t), 256); }
static WorkList worklist_at(void* base, int B) {
  WorkList w;
  w.blkcum = reinterpret_cast<int32_t*>(base);
  w.perm = w.blkcum + (B + 1);
  w.scum = w.perm + B;
  w.cus = w.scum + (B + 1);
  w.status = w.cus + (B + 1);
  return w;
}


typedef int (*bwd_dispatch_fn)(const BwdParams&, int, int, int, hipStream_t, int, bool, int*);

static bwd_dispatch_fn bwd_table(int dtype, int D) {
  if (dtype == FST_BF16) {
    switch (D) {
      case 16: return bwd_dispatch_bf16_16;
      case 32: return bwd_dispatch_bf16_32;
      case 48: return bwd_dispatch_bf16_48;
      case 64: return bwd_dispatch_bf16_64;
    }
  } else if (dtype == FST_F32) {
    switch (D) {
      case 16: return bwd_dispatch_f32_16;
      case 32: return bwd_dispatch_f32_32;
      case 48: return bwd_dispatch_f32_48;
      case 64: return bwd_dispatch_f32_64;
    }
  }
  return nullptr;
}

// dW / db from the per-block partials of the rows kernel, in two fixed-order
// stages so the result does not depend on scheduling: stage 1 sums runs of
// kRedSeg consecutive blocks per column (coalesced over the columns), stage
// 2 sums the run totals in order.
constexpr int kRedSeg = 64;

__global__ __launch_bounds__(256) void dw_reduce_seg_kernel(const float* part, const int32_t* blkcum, int B,
                                                            int ncol, float* seg) {
  const int nblk = blkcum[B];
  const int col = blockIdx.x * 256 + threadIdx.x;
  if (col >= ncol) return;
  const long w0 = (long)blockIdx.y * kRedSeg;
  const long w1 = w0 + kRedSeg < nblk ? w0 + kRedSeg : nblk;
  float acc = 0.f;
#pragma unroll 8
  for (long w = w0; w < w1; ++w) acc += part[w * ncol + col];
  seg[(long)blockIdx.y * ncol + col] = acc;
}

// Stage 2: a workgroup per 64 columns; thread (q, c) sums runs q, q + 4, ...
// of column c, and the four partial sums are added in the order q = 0..3.
__global__ __launch_bounds__(256) void dw_reduce_final_kernel(const float* seg, int nseg, int DC, int D, int use_e,
                                                              float* dw, float* db) {
  __shared__ float part[4][64];
  const int c = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int e = blockIdx.x * 64 + c;
  float acc = 0.f;
  if (use_e && e < DC + D) {
#pragma unroll 8
    for (int s = q; s < nseg; s += 4) acc += seg[(long)s * (DC + D) + e];
  }
  part[q][c] = acc;
  __syncthreads();
  if (q != 0 || e >= DC + D) return;
  acc = ((part[0][c] + part[1][c]) + part[2][c]) + part[3][c];
  if (e < DC)
    dw[e] = acc;
  else if (db)
    db[e - DC] = acc;
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float* p, int n) {
  for (int i = threadIdx.x; i < n; i += 256) p[i] = 0.f;
}

struct BwdLayout {
  int rows_r, rows_c;   // rows (keys) per workgroup of the rows / cols kernels
  long grid_r, grid_c;
  size_t off_bc_r, off_bc_c, off_vp, off_u, off_wt, off_qt, off_dob, off_dsum, off_lsez, off_part, off_seg, total;
  long nseg;  // stage-1 runs of the dW reduction
};

static int bwd_layout(int dtype, int flags, int B, int H, int L, int T, int D, int C, BwdLayout& lay) {
  bwd_dispatch_fn fn = bwd_table(dtype, D);
  BwdParams dummy;
  std::memset(&dummy, 0, sizeof(dummy));
  dummy.flags = flags;  // the queries resolve the plan bits
  const int HP = head_padding(H), HPR = rows_head_padding(dtype, flags, H, D, C);
  if (fn(dummy, 0, HPR, C, nullptr, 0, true, &lay.rows_r) != FST_OK || lay.rows_r <= 0) return FST_EUNSUPPORTED;
  if (fn(dummy, 1, HP, C, nullptr, 0, true, &lay.rows_c) != FST_OK || lay.rows_c <= 0) return FST_EUNSUPPORTED;
  const bool packed = flags & FST_PACKED;
  const long rows = packed ? (long)T : (long)B * L;
  const long B8 = (B + 7) / 8 * 8;
  lay.grid_r = packed ? ((long)T + lay.rows_r - 1) / lay.rows_r + B : B8 * ((L + lay.rows_r - 1) / lay.rows_r);
  lay.grid_c = packed ? ((long)T + lay.rows_c - 1) / lay.rows_c + B : B8 * ((L + lay.rows_c - 1) / lay.rows_c);
  const size_t esz = dtype == FST_BF16 ? 2 : 4;
  size_t off = 0;
  lay.off_bc_r = off;
  off += blkcum_bytes(B);
  lay.off_bc_c = off;
  off += blkcum_bytes(B);
  // The rows kernel's padding-last schedule (bf16, padded).
  lay.off_vp = off;
  off += align_up((size_t)(8 * ((B + 7) / 8) + 1) * sizeof(int32_t), 256);
  // u and w~ hold whole 16-row tiles of each event (the bf16 kernels' row-group
  // layout): at most B ceil(L / 16) tiles padded, T / 16 + B packed.
  const long rows_uw = packed ? ((long)(T + 15) / 16 + B) * 16 : (long)B * ((L + 15) / 16) * 16;
  lay.off_u = off;
  off += align_up((size_t)(rows_uw > rows ? rows_uw : rows) * H * C * esz, 256);
  lay.off_wt = off;
  off += align_up((size_t)(rows_uw > rows ? rows_uw : rows) * H * C * esz, 256);
  lay.off_qt = off;
  if (dtype == FST_BF16) off += align_up((size_t)rows * H * D * esz, 256);
  lay.off_dob = off;
  off += align_up((size_t)rows * H * 4, 256);
  lay.off_dsum = off;
  off += align_up((size_t)rows * H * 4, 256);
  lay.off_lsez = off;
  off += align_up((size_t)rows * H * 4, 256);
  // The dW / db partials (one per rows-kernel workgroup) are sized for
  // 16-row workgroups, the smallest of any plan, so that the workspace a
  // caller sizes without plan bits serves every plan.
  const long grid16 = packed ? ((long)T + 15) / 16 + B : B8 * ((L + 15) / 16);
  const long nseg16 = (grid16 + kRedSeg - 1) / kRedSeg;
  lay.off_part = off;
  off += align_up((size_t)(grid16 > 0 ? grid16 : 0) * (D * C + D) * 4, 256);
  lay.nseg = lay.grid_r > 0 ? (lay.grid_r + kRedSeg - 1) / kRedSeg : 0;
  lay.off_seg = off;
  off += align_up((size_t)(nseg16 > 0 ? nseg16 : 0) * (D * C + D) * 4, 256);
  lay.total = off;
  return FST_OK;
}

}  // namespace fst

using namespace fst;

extern "C" {

const char* fst_last_error(void) { return g_last_error; }

#ifndef FST_BUILD_ID
#define FST_BUILD_ID "unknown"
#endif
const char* fst_version(void) { return "flash-spacetime-gfx950 0.3.0 abi 2 build " FST_BUILD_ID; }

void fst_frequencies(int C, float* out) {
  if (C > 0 && C <= 64 && C % 2 == 0 && out) frequencies(C, out);
}

int fst_max_event_len(int dtype, int flags, int H, int D, int C) {
  if (check_common(dtype, flags & ~FST_PLAN_MASK, 0, H, 0, 0, D, C) != FST_OK) return 0;
  return max_event_len(dtype, flags, H, D, C);
}

int fst_plans(int dtype, int H, int D, int C) {
  if (check_common(dtype, 0, 0, H, 0, 0, D, C) != FST_OK) return 0;
  return shape_plans(dtype, H, D, C);
}

int fst_plan_supported(int dtype, int H, int D, int C, int plan) {
  if (plan & ~FST_PLAN_MASK) return 0;
  if (check_common(dtype, plan, 0, H, 0, 0, D, C) != FST_OK) return 0;
  int rows = 0;
  FwdParams dummy;
  std::memset(&dummy, 0, sizeof(dummy));
  dummy.flags = plan;
  if (fwd_table(dtype, D)(dummy, head_padding(H), C, nullptr, 0, true, &rows) != FST_OK || rows <= 0) return 0;
  BwdLayout lay;
  return bwd_layout(dtype, plan, 1, H, 16, 0, D, C, lay) == FST_OK;
}

int fst_supported(int dtype, int H, int D, int C) {
  if (check_common(dtype, 0, 0, H, 0, 0, D, C) != FST_OK) return 0;
  int rows = 0;
  FwdParams dummy;
  std::memset(&dummy, 0, sizeof(dummy));
  if (fwd_table(dtype, D)(dummy, head_padding(H), C, nullptr, 0, true, &rows) != FST_OK || rows <= 0) return 0;
  BwdLayout lay;
  return bwd_layout(dtype, 0, 1, H, 16, 0, D, C, lay) == FST_OK;
}

size_t fst_forward_workspace_bytes(int dtype, int flags, int B, int H, int L, int T, int D, int C) {
  (void)dtype;
  (void)flags;
  (void)H;
  (void)L;
  (void)T;
  (void)D;
  (void)C;
  return blkcum_bytes(B < 0 ? 0 : B);
}

int fst_forward_phases(int phases, int dtype, int flags, int B, int H, int L, int T, int D, int C, const void* q,
                       const void* k, const void* v, const float* pos4, const float* weight, const float* bias,
                       const int32_t* lens, float scale, void* out, float* lse, void* workspace,
                       size_t workspace_bytes, void* stream) {
  g_last_error[0] = 0;
  if (phases & ~FST_FWD_ALL) return fail(FST_EINVAL, "unknown forward phase bits 0x%x", phases);
  int rc = check_common(dtype, flags, B, H, L, T, D, C);
  if (rc != FST_OK) return rc;
  const bool packed = flags & FST_PACKED;
  const bool use_w = flags & (FST_ATTN_BIAS | FST_ACT_BIAS);
  const long rows_total = packed ? (long)T : (long)B * L;
  if (B == 0 || rows_total == 0) return FST_OK;
  if (!q || !k || !v || !lens || !out || !lse) return fail(FST_EINVAL, "null tensor pointer");
  if (use_w && (!pos4 || !weight)) return fail(FST_EINVAL, "pos4 and weight are required when a bias flag is set");
  if (!std::isfinite(scale)) return fail(FST_EINVAL, "scale must be finite");
  const size_t need = fst_forward_workspace_bytes(dtype, flags, B, H, L, T, D, C);
  if (!workspace || workspace_bytes < need)
    return fail(FST_EWORKSPACE, "workspace of %zu bytes is smaller than the %zu required", workspace_bytes, need);

  fwd_dispatch_fn fn = fwd_table(dtype, D);
  const int HP = head_padding(H);
  FwdParams prm;
  std::memset(&prm, 0, sizeof(prm));
  prm.flags = flags;  // the query resolves the plan bits
  int rows = 0;
  rc = fn(prm, HP, C, nullptr, 0, true, &rows);
  if (rc != FST_OK || rows <= 0)
    return fail(FST_EUNSUPPORTED, "no compiled forward kernel for dtype=%d H=%d D=%d C=%d with plan bits 0x%x", dtype,
                H, D, C, flags & FST_PLAN_MASK);

  const WorkList wl = worklist_at(workspace, B);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (phases & FST_PHASE_WORKLIST) {
    if (launch_worklist(lens, packed, B, L, T, rows, wl.blkcum, 0, nullptr, wl.perm, wl.scum, nullptr, wl.cus,
                        wl.status, st) != FST_OK)
      return fail(FST_ELAUNCH, "work-list kernel launch failed");
  }

  if (!(phases & FST_PHASE_FWD)) return FST_OK;

  prm.ev.lens = packed ? wl.cus : lens;
  prm.ev.blkcum = wl.blkcum;
  prm.ev.perm = wl.perm;
  prm.ev.scum = packed ? wl.scum : nullptr;
  prm.ev.status = wl.status;
  prm.ev.max_len = max_event_len(dtype, flags, H, D, C);
  prm.ev.pos4 = reinterpret_cast<const float4*>(pos4);
  prm.ev.B = B;
  prm.ev.H = H;
  prm.ev.L = L;
  prm.ev.T = T;
  prm.ev.packed = packed ? 1 : 0;
  prm.ev.tokmajor = (packed || (flags & FST_TOKEN_MAJOR)) ? 1 : 0;
  prm.ev.xmul = (flags & FST_QKV_INTERLEAVED) ? 3 : 1;
  prm.H = H;
  prm.flags = flags;
  prm.scale = scale;
  prm.q = q;
  prm.k = k;
  prm.v = v;
  prm.weight = weight;
  prm.bias = bias;
  prm.out = out;
  prm.lse = lse;
  freq_table(C, prm.freq);
  // Padded grids cover ceil(B / 8) * 8 events (the tile kernels' schedule
  // deals events to the eight XCDs); workgroups without work exit at once.
  const long grid = packed ? ((long)T + rows - 1) / rows + B : (long)((B + 7) / 8 * 8) * ((L + rows - 1) / rows);
  if (grid > 0x7fffffffL) return fail(FST_EUNSUPPORTED, "problem too large for one launch");
  rc = fn(prm, HP, C, st, (int)grid, false, &rows);
  if (rc != FST_OK) return fail(rc, "forward kernel launch failed (%s)", hipGetErrorString(hipGetLastError()));
  return FST_OK;
}

// ---------------------------------------------------------------------------
// Allocation-free forward. The forward's only scratch is its work list
// (blkcum_bytes(B)), which fst_forward_noalloc keeps in a file-scope device
// array sized for kNoAllocMaxEvents events. Each device holds its own copy;
// in host code `scratch` names a host-side stand-in, so its device address
// is resolved once per device with hipGetSymbolAddress (with that device
// current) and only that address is handed to the kernels.
// ---------------------------------------------------------------------------
}  // extern "C"

namespace fst {
constexpr int kNoAllocMaxEvents = 65536;
constexpr size_t kNoAllocBytes = (size_t)(4 * kNoAllocMaxEvents + 4) * sizeof(int32_t);
static __device__ __align__(256) unsigned char scratch[(kNoAllocBytes + 255) / 256 * 256];
constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// The device address of `scratch` on the device of `stream`, which must be
// the current device: hipGetSymbolAddress resolves the current device's copy
// (nullptr and an error message on failure, with *rc the status to return).
static void* scratch_for_stream(hipStream_t stream, int* rc) {
  int dev = -1, sdev = -1;
  *rc = FST_ELAUNCH;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(FST_ELAUNCH, "no current HIP device (or device index %d beyond %d)", dev, kMaxDevices);
    return nullptr;
  }
  if (hipStreamGetDevice(stream, &sdev) != hipSuccess) {
    fail(FST_ELAUNCH, "hipStreamGetDevice failed");
    return nullptr;
  }
  if (sdev != dev) {
    *rc = FST_EINVAL;
    fail(FST_EINVAL, "the stream belongs to device %d but device %d is current: make the stream's device current",
         sdev, dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (rc != hipSuccess || !ptr) {
      fail(FST_ELAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(rc));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}
}  // namespace fst

extern "C" {

int fst_forward_noalloc(int dtype, int flags, int B, int H, int L, int T, int D, int C, const void* q,
                        const void* k, const void* v, const float* pos4, const float* weight, const float* bias,
                        const int32_t* lens, float scale, void* out, float* lse, void* stream) {
  g_last_error[0] = 0;
  if (B > kNoAllocMaxEvents)
    return fail(FST_EUNSUPPORTED, "fst_forward_noalloc takes at most %d events, got %d (use fst_forward)",
                kNoAllocMaxEvents, B);
  const int rc = check_common(dtype, flags, B, H, L, T, D, C);
  if (rc != FST_OK) return rc;
  const size_t need = fst_forward_workspace_bytes(dtype, flags, B, H, L, T, D, C);
  if (need > sizeof(scratch)) return fail(FST_EUNSUPPORTED, "work list of %zu bytes exceeds the %zu-byte scratch",
                                          need, sizeof(scratch));
  const bool packed = flags & FST_PACKED;
  if (B == 0 || (packed ? (long)T : (long)B * L) == 0) return FST_OK;
  int src = FST_OK;
  void* ws = scratch_for_stream(reinterpret_cast<hipStream_t>(stream), &src);
  if (!ws) return src;
  return fst_forward_phases(FST_FWD_ALL, dtype, flags, B, H, L, T, D, C, q, k, v, pos4, weight, bias, lens, scale,
                            out, lse, ws, sizeof(scratch), stream);
}

int fst_forward(int dtype, int flags, int B, int H, int L, int T, int D, int C, const void* q, const void* k,
                const void* v, const float* pos4, const float* weight, const float* bias, const int32_t* lens,
                float scale, void* out, float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  return fst_forward_phases(FST_FWD_ALL, dtype, flags, B, H, L, T, D, C, q, k, v, pos4, weight, bias, lens, scale,
                            out, lse, workspace, workspace_bytes, stream);
}

size_t fst_backward_workspace_bytes(int dtype, int flags, int B, int H, int L, int T, int D, int C) {
  if (check_common(dtype, flags, B, H, L, T, D, C) != FST_OK) return 0;
  BwdLayout lay;
  if (bwd_layout(dtype, flags, B, H, L, T, D, C, lay) != FST_OK) return 0;
  return lay.total;
}

int fst_backward_phases(int phases, int dtype, int flags, int B, int H, int L, int T, int D, int C, const void* q,
                        const void* k, const void* v, const float* pos4, const float* weight, const float* bias,
                        const int32_t* lens, const float* lse, const void* grad_out, const void* out, float scale,
                        void* dq, void* dk, void* dv, float* dweight, float* dbias, float* rowsum, void* workspace,
                        size_t workspace_bytes, void* stream) {
  g_last_error[0] = 0;
  if (phases & ~FST_BWD_ALL) return fail(FST_EINVAL, "unknown backward phase bits 0x%x", phases);
  int rc = check_common(dtype, flags, B, H, L, T, D, C);
  if (rc != FST_OK) return rc;
  const bool packed = flags & FST_PACKED;
  const bool use_w = flags & (FST_ATTN_BIAS | FST_ACT_BIAS);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const long rows_total = packed ? (long)T : (long)B * L;
  if (!dweight) return fail(FST_EINVAL, "dweight is required");
  if (B == 0 || rows_total == 0) {
    if (phases & FST_PHASE_REDUCE) {
      hipLaunchKernelGGL(fill_zero_kernel, dim3(1), dim3(256), 0, st, dweight, D * C);
      if (dbias) hipLaunchKernelGGL(fill_zero_kernel, dim3(1), dim3(256), 0, st, dbias, D);
      if (hipGetLastError() != hipSuccess) return fail(FST_ELAUNCH, "zero fill launch failed");
    }
    return FST_OK;
  }
  if (!q || !k || !v || !lens || !lse || !grad_out || !dq || !dk || !dv)
    return fail(FST_EINVAL, "null tensor pointer");
  if (use_w && (!pos4 || !weight)) return fail(FST_EINVAL, "pos4 and weight are required when a bias flag is set");
  if (!std::isfinite(scale)) return fail(FST_EINVAL, "scale must be finite");
  BwdLayout lay;
  if (bwd_layout(dtype, flags, B, H, L, T, D, C, lay) != FST_OK)
    return fail(FST_EUNSUPPORTED, "no compiled backward for dtype=%d H=%d D=%d C=%d", dtype, H, D, C);
  if (!workspace || workspace_bytes < lay.total)
    return fail(FST_EWORKSPACE, "workspace of %zu bytes is smaller than the %zu required", workspace_bytes, lay.total);
  if (lay.grid_r > 0x7fffffffL || lay.grid_c > 0x7fffffffL) return fail(FST_EUNSUPPORTED, "problem too large");

  unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
  const WorkList wr = worklist_at(ws + lay.off_bc_r, B), wc = worklist_at(ws + lay.off_bc_c, B);
  // The bf16 rows kernel's padding-last schedule (16-row tiles, padded events).
  int32_t* vp = (dtype == FST_BF16 && !packed && lay.rows_r == 16) ? reinterpret_cast<int32_t*>(ws + lay.off_vp)
                                                                    : nullptr;
  if (phases & FST_PHASE_WORKLIST) {
    if (launch_worklist(lens, packed, B, L, T, lay.rows_r, wr.blkcum, lay.rows_c, wc.blkcum, wr.perm, wr.scum,
                        wc.scum, wr.cus, wr.status, st, vp) != FST_OK)
      return fail(FST_ELAUNCH, "work-list kernel launch failed");
  }

  BwdParams prm;
  std::memset(&prm, 0, sizeof(prm));
  prm.ev.lens = packed ? wr.cus : lens;
  prm.ev.blkcum = wr.blkcum;
  prm.ev.perm = wr.perm;
  prm.ev.scum = packed ? wr.scum : nullptr;
  prm.ev.vp = vp;
  prm.ev.status = wr.status;
  prm.ev.max_len = max_event_len(dtype, flags, H, D, C);
  prm.ev.pos4 = reinterpret_cast<const float4*>(pos4);
  prm.ev.B = B;
  prm.ev.H = H;
  prm.ev.L = L;
  prm.ev.T = T;
  prm.ev.packed = packed ? 1 : 0;
  prm.ev.tokmajor = (packed || (flags & FST_TOKEN_MAJOR)) ? 1 : 0;
  prm.ev.xmul = (flags & FST_QKV_INTERLEAVED) ? 3 : 1;
  prm.blkcum_cols = wc.blkcum;
  prm.scum_cols = packed ? wc.scum : nullptr;
  prm.H = H;
  prm.flags = flags;
  prm.scale = scale;
  prm.q = q;
  prm.k = k;
  prm.v = v;
  prm.dout = grad_out;
  prm.out = dtype == FST_BF16 ? out : nullptr;
  prm.weight = weight;
  prm.bias = bias;
  prm.lse = lse;
  prm.u = ws + lay.off_u;
  prm.wt = ws + lay.off_wt;
  prm.qt = ws + lay.off_qt;
  prm.dob = reinterpret_cast<float*>(ws + lay.off_dob);
  prm.dsum = reinterpret_cast<float*>(ws + lay.off_dsum);
  prm.lse_z = reinterpret_cast<float*>(ws + lay.off_lsez);
  prm.dw_part = reinterpret_cast<float*>(ws + lay.off_part);
  prm.dq = dq;
  prm.dk = dk;
  prm.dv = dv;
  prm.rowsum = rowsum;
  prm.dweight = dweight;
  prm.dbias = dbias;
  freq_table(C, prm.freq);

  bwd_dispatch_fn fn = bwd_table(dtype, D);
  const int HP = head_padding(H), HPR = rows_head_padding(dtype, flags, H, D, C);
  int dummy_rows = 0;
  if (phases & FST_PHASE_BWD_ROWS) {
    rc = fn(prm, 0, HPR, C, st, (int)lay.grid_r, false, &dummy_rows);
    if (rc != FST_OK) return fail(rc, "backward rows kernel launch failed");
  }
  if (phases & FST_PHASE_BWD_COLS) {
    rc = fn(prm, 1, HP, C, st, (int)lay.grid_c, false, &dummy_rows);
    if (rc != FST_OK) return fail(rc, "backward cols kernel launch failed");
  }
  if (phases & FST_PHASE_REDUCE) {
    const int DC = D * C;
    const int ncol = DC + D;
    float* seg = reinterpret_cast<float*>(ws + lay.off_seg);
    if (lay.nseg > 65535) return fail(FST_EUNSUPPORTED, "problem too large for the dW reduction");
    if (use_w && lay.nseg > 0)
      hipLaunchKernelGGL(dw_reduce_seg_kernel, dim3((ncol + 255) / 256, (unsigned)lay.nseg), dim3(256), 0, st,
                         prm.dw_part, wr.blkcum, B, ncol, seg);
    hipLaunchKernelGGL(dw_reduce_final_kernel, dim3((ncol + 63) / 64), dim3(256), 0, st, seg, (int)lay.nseg, DC,
                       D, use_w ? 1 : 0, dweight, dbias);
    if (hipGetLastError() != hipSuccess) return fail(FST_ELAUNCH, "dW reduction launch failed");
  }
  return FST_OK;
}

int fst_backward(int dtype, int flags, int B, int H, int L, int T, int D, int C, const void* q, const void* k,
                 const void* v, const float* pos4, const float* weight, const float* bias, const int32_t* lens,
                 const float* lse, const void* grad_out, const void* out, float scale, void* dq, void* dk, void* dv,
                 float* dweight, float* dbias, float* rowsum, void* workspace, size_t workspace_bytes, void* stream) {
  return fst_backward_phases(FST_BWD_ALL, dtype, flags, B, H, L, T, D, C, q, k, v, pos4, weight, bias, lens, lse,
                             grad_out, out, scale, dq, dk, dv, dweight, dbias, rowsum, workspace, workspace_bytes,
                             stream);
}

}  // extern "C"
