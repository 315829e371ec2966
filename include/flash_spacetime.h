/*
 * flash_spacetime.h -- C ABI of the MI355X (gfx950) flash-spacetime library.
 *
 * Spacetime-interval-biased attention (sevmag/flash-spacetime) as plain C
 * entry points over caller-owned device buffers. No entry point allocates,
 * frees or synchronises: every buffer, including the scratch workspace
 * whose size the *_workspace_bytes queries return, belongs to the caller,
 * and all work is enqueued on the caller's HIP stream.
 *
 * Layouts (all contiguous, row-major):
 *   padded : q, k, v, out, dq, dk, dv  [B, H, L, D]   lse, rowsum [B, H, L]
 *            pos4 [B, L, 4] fp32 (x, y, z, t), lens = seqlens [B] int32
 *            (valid tokens of event b are 0 .. seqlens[b]-1)
 *   padded, FST_TOKEN_MAJOR :
 *            q, k, v, out, grad_out, dq, dk, dv  [B, L, H, D]
 *            lse, rowsum [B, L, H]; pos4 and lens as padded
 *   packed : q, k, v, out, dq, dk, dv  [T, H, D]      lse, rowsum [T, H]
 *            pos4 [T, 4] fp32, lens = cu_seqlens [B+1] int32 (cu[0] = 0,
 *            cu[B] = T)
 *   FST_QKV_INTERLEAVED (with FST_TOKEN_MAJOR or FST_PACKED): q, k, v are
 *            the three slots of one [B, L, 3, H, D] / [T, 3, H, D] tensor
 *            (q = its base, k = base + H*D, v = base + 2*H*D elements), and
 *            dq, dk, dv likewise of one gradient tensor; out, grad_out,
 *            lse and rowsum keep the [B, L, H, D] / [T, H, D] layout.
 *   weight [D, C] fp32 (nn.Linear layout), bias [D] fp32 or NULL.
 *   dtype FST_BF16: q, k, v, out, grad_out, dq, dk, dv are bfloat16;
 *   dtype FST_F32 : they are float32. lse, pos4, weight, bias, dweight,
 *   dbias, rowsum are float32 in both.
 *
 * Supported shapes: 1 <= H <= 16, D in {16, 32, 48, 64}, C in {16, 32, 48,
 * 64} (C even, sin/cos halves); see fst_supported(). Callers run more heads
 * as head groups of their own (the Python operators take any H). One event
 * may hold at most fst_max_event_len() tokens: the kernels address an
 * event's rows of all heads with 32-bit byte offsets. Padded calls beyond
 * that return FST_EUNSUPPORTED; a packed event beyond it (its length lives on
 * the device) gets NaN in its rows of out and lse (forward) or dq, dk, dv,
 * rowsum and in dweight / dbias (backward) instead of results.
 *
 * Malformed packed offsets (cu_seqlens[0] != 0, a decreasing offset, or
 * cu_seqlens[B] > T) never make the kernels access memory outside the
 * tensors or the workspace: the work list runs on their running maximum
 * clamped to [0, T] and every row the kernels write gets NaN (as above).
 * Tokens past cu_seqlens[B] < T belong to no event and are not written.
 *
 * Return value: 0 on success, a negative FST_E* code otherwise; the message
 * of the last failure on the calling thread is in fst_last_error().
 */
#ifndef FLASH_SPACETIME_H
#define FLASH_SPACETIME_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum fst_dtype { FST_BF16 = 0, FST_F32 = 1 };

enum fst_flags {
  FST_ATTN_BIAS = 1, /* add qt_i . R_ij to the logits (use_attn_bias)        */
  FST_ACT_BIAS = 2,  /* add sum_j P_ij R_ij to the output (use_activation_bias) */
  FST_PACKED = 4,    /* packed [T, H, D] layout with cu_seqlens              */
  FST_TOKEN_MAJOR = 8, /* padded tensors stored [B, L, H, D] (vectors [B, L, H]):
                         the heads-first views of a [B, L, H*D] projection
                         (reference.py:187-196 split_heads) read in place.
                         No reference counterpart: the reference makes them
                         contiguous [B, H, L, D] first (forward.py:274).    */
  FST_QKV_INTERLEAVED = 16, /* q, k, v (and dq, dk, dv) interleaved per token as
                              one fused projection's [.., 3, H, D] output; see
                              Layouts. No reference counterpart (the reference
                              takes three separate tensors, forward.py:481). */
  /* Plan bits: a choice among compiled variants of the kernels, for callers
   * that time them. Each group below is one knob of one kernel; at most one
   * bit of a group may be set, and a group left empty takes the library's
   * static choice. fst_plans() lists the bits compiled for a shape and
   * fst_plan_supported() whether one combination of them is.
   * Variants of the occupancy, wave, K/V-staging and tile-height groups
   * compute every output row with the same arithmetic: out, lse, dq, dk, dv
   * and rowsum are the same bit for bit, and dweight / dbias differ only in
   * the order in which their fp32 partial sums are added. The key-chunk
   * groups move the points where the online softmax rescales and the order
   * of the sums over keys, and the pass group forms D online or in a first
   * pass, so their results agree to rounding.
   * No reference counterpart: the reference's Triton kernels take fixed tile
   * constants (_tiles.py), are not autotuned (README.md:86-95), and its
   * launchers' block_m / block_n / num_warps arguments (forward.py:233-236,
   * backward.py:501-504) select those constants; the Python operators map
   * them onto the tile-height, key-chunk and wave groups. */
  /* bf16 forward: workgroups per CU */
  FST_PLAN_FWD_OCC2 = 1 << 8,
  FST_PLAN_FWD_OCC3 = 1 << 9,
  /* bf16 backward rows kernel: waves per workgroup and workgroups per CU */
  FST_PLAN_ROWS_W4 = 1 << 10,   /* four waves, two workgroups per CU               */
  FST_PLAN_ROWS_W8 = 1 << 11,   /* eight waves, one per CU (heads padded to 8k)    */
  FST_PLAN_ROWS_W8X2 = 1 << 14, /* eight waves, two per CU (four waves per SIMD)   */
  /* bf16 backward cols kernel: workgroups per CU */
  FST_PLAN_COLS_OCC2 = 1 << 12,
  FST_PLAN_COLS_OCC3 = 1 << 13,
  /* bf16 backward rows kernel: where a key chunk's K and V rows are held */
  FST_PLAN_ROWS_KV_REG = 1 << 15, /* registers, loaded a chunk ahead            */
  FST_PLAN_ROWS_KV_LDS = 1 << 16, /* LDS, by direct loads (D a multiple of 32)  */
  /* forward: keys per chunk (bf16 and float32) */
  FST_PLAN_FWD_KC16 = 1 << 17,
  FST_PLAN_FWD_KC32 = 1 << 18,
  /* float32 forward: query rows per workgroup (tile height); one group with
   * FST_PLAN_FWD_W8 */
  FST_PLAN_FWD_T16 = 1 << 19,
  FST_PLAN_FWD_T32 = 1 << 20,
  FST_PLAN_FWD_T64 = 1 << 21,
  /* float32 backward: rows (rows kernel) and keys (cols kernel) per
   * workgroup; one group with FST_PLAN_BWD_W8 */
  FST_PLAN_BWD_T16 = 1 << 22,
  FST_PLAN_BWD_T32 = 1 << 23,
  FST_PLAN_BWD_T64 = 1 << 24,
  /* float32 backward: keys (rows kernel) and rows (cols kernel) per chunk */
  FST_PLAN_BWD_KC16 = 1 << 25,
  FST_PLAN_BWD_KC32 = 1 << 26,
  /* float32 backward rows kernel: passes over the keys (one, with D formed
   * online and the accumulators corrected as it moves; or two, D first) */
  FST_PLAN_BWD_PASS1 = 1 << 27,
  FST_PLAN_BWD_PASS2 = 1 << 28,
  /* float32: a 16-row tile served by eight waves (the T16 tile of four
   * waves, with each wave's heads and rows halved) */
  FST_PLAN_FWD_W8 = 1 << 29,
  FST_PLAN_BWD_W8 = 1 << 30,
  FST_PLAN_MASK = 0x7fffff00
};

/* Phases of one operator call, for callers that time or schedule them
 * separately (the one-shot entry points run all of them, in this order).
 * The work list (per-event row-block prefix sums) is written into the
 * workspace by the first phase and read by the later ones. */
enum fst_phase {
  FST_PHASE_WORKLIST = 1, /* per-event row blocks -> workspace (tiny kernel)   */
  FST_PHASE_FWD = 2,      /* forward kernel                                   */
  FST_PHASE_BWD_ROWS = 4, /* backward rows kernel: D, dq, H, G, dW/db partials */
  FST_PHASE_BWD_COLS = 8, /* backward cols kernel: dk, dv                     */
  FST_PHASE_REDUCE = 16,  /* ordered sum of the dW / db partials              */
  FST_FWD_ALL = FST_PHASE_WORKLIST | FST_PHASE_FWD,
  FST_BWD_ALL = FST_PHASE_WORKLIST | FST_PHASE_BWD_ROWS | FST_PHASE_BWD_COLS | FST_PHASE_REDUCE
};

enum fst_status {
  FST_OK = 0,
  FST_EINVAL = -1,       /* bad argument (shape, pointer, flag)             */
  FST_EUNSUPPORTED = -2, /* valid request outside the compiled shape set    */
  FST_EWORKSPACE = -3,   /* workspace smaller than *_workspace_bytes()       */
  FST_ELAUNCH = -4       /* HIP launch error                                 */
};

/* 1 if (dtype, H, D, C) has compiled forward and backward kernels, else 0
 * (float32 at D = C = 64 has them up to H = 8; callers split more heads
 * into groups, as the Python operators do).
 * No reference counterpart: the Triton reference JIT-compiles per shape and
 * raises ValueError for C outside {16, 32, 48} (forward.py:261-265). */
int fst_supported(int dtype, int H, int D, int C);

/* The FST_PLAN_* bits compiled for (dtype, H, D, C): a bit is set when its
 * variant exists for the shape in some combination with the other groups
 * (0 for unsupported shapes).
 * No reference counterpart (see the plan bits above). */
int fst_plans(int dtype, int H, int D, int C);

/* 1 if the combination `plan` of FST_PLAN_* bits (at most one per group;
 * the empty groups take the static choice) is compiled for (dtype, H, D, C)
 * in both the forward and the backward, else 0.
 * No reference counterpart (see the plan bits above). */
int fst_plan_supported(int dtype, int H, int D, int C, int plan);

/* Scratch bytes fst_forward needs for these sizes (rows = B*L padded, T packed). */
size_t fst_forward_workspace_bytes(int dtype, int flags, int B, int H, int L, int T,
                                   int D, int C);

/* Fused forward. Writes out (pad rows exactly 0) and lse (log-sum-exp of the
 * logits without the row-constant qt.b term; 0 on pad rows).
 * Replaces flash_spacetime_forward (reference forward.py:222-346) together
 * with the Triton kernel launch it makes (forward.py:306-331); the o2
 * epilogue (forward.py:333-346) is fused into the kernel. */
int fst_forward(int dtype, int flags, int B, int H, int L, int T, int D, int C,
                const void* q, const void* k, const void* v, const float* pos4,
                const float* weight, const float* bias, const int32_t* lens,
                float scale, void* out, float* lse, void* workspace,
                size_t workspace_bytes, void* stream);

/* fst_forward with no workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. The
 * work list lives in a file-scope device array of the library sized for at
 * most 65536 events (B > 65536 returns FST_EUNSUPPORTED); each GPU holds its
 * own copy, about 1 MiB, until the process ends. The stream's device must
 * be the current device (else FST_EINVAL): the first call on a device
 * resolves the array's address there, and every call uses the current
 * device's copy. No call allocates, frees or synchronises. Every call on one GPU shares
 * that GPU's array, so calls that overlap on one GPU (concurrent streams or
 * threads) race: serialise them. Results are bitwise those of fst_forward. */
int fst_forward_noalloc(int dtype, int flags, int B, int H, int L, int T, int D, int C,
                        const void* q, const void* k, const void* v, const float* pos4,
                        const float* weight, const float* bias, const int32_t* lens,
                        float scale, void* out, float* lse, void* stream);

/* fst_forward restricted to the given phases (FST_PHASE_WORKLIST,
 * FST_PHASE_FWD), for callers that time or schedule the phases; no
 * reference counterpart beyond forward.py:306-331 (the launch itself). */
int fst_forward_phases(int phases, int dtype, int flags, int B, int H, int L, int T, int D,
                       int C, const void* q, const void* k, const void* v,
                       const float* pos4, const float* weight, const float* bias,
                       const int32_t* lens, float scale, void* out, float* lse,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Scratch bytes fst_backward needs. */
size_t fst_backward_workspace_bytes(int dtype, int flags, int B, int H, int L, int T,
                                    int D, int C);

/* Deterministic backward from the saved lse. Writes dq, dk, dv (pad rows 0),
 * dweight [D, C] and, when bias != NULL, dbias [D] (all float32 for the
 * weight-side). rowsum (nullable, float32 like lse) receives sum_j dS_ij,
 * which the normalised softmax row term makes zero up to rounding: float32
 * sums the dS values its products were fed (corrections included); bf16
 * writes N - D Z from the float32 sums N = sum P dP, Z = sum P that define
 * D = N / Z, which is zero up to one rounding by construction and so says
 * nothing about the bf16 dS values (the tests measure those through dq with
 * every key of an event equal).
 * out (nullable) is the forward's output, laid out as grad_out. With bf16
 * operands the rows kernel then forms dS against a reference D taken from it
 * (dO . (out - b), b with FST_ACT_BIAS) and corrects its sums to the
 * in-kernel D = sum P dP / sum P once, after its last key chunk, instead of
 * after every chunk; D itself, and so every gradient up to rounding, is the
 * same either way. Ignored for float32.
 * Replaces flash_spacetime_backward (reference backward.py:488-630): the
 * host prologue (:526-556), both Triton kernels (:589-598) and the host
 * epilogue (:600-630); `out` has no counterpart there (the reference's
 * launcher does not take the output). */
int fst_backward(int dtype, int flags, int B, int H, int L, int T, int D, int C,
                 const void* q, const void* k, const void* v, const float* pos4,
                 const float* weight, const float* bias, const int32_t* lens,
                 const float* lse, const void* grad_out, const void* out, float scale,
                 void* dq, void* dk, void* dv, float* dweight, float* dbias, float* rowsum,
                 void* workspace, size_t workspace_bytes, void* stream);

/* fst_backward restricted to the given phases (FST_PHASE_WORKLIST,
 * FST_PHASE_BWD_ROWS, FST_PHASE_BWD_COLS, FST_PHASE_REDUCE): the rows and cols
 * kernels are the counterparts of the reference's two Triton launches
 * (backward.py:589-598), the reduce phase of its dW/db epilogue
 * (backward.py:607-622). */
int fst_backward_phases(int phases, int dtype, int flags, int B, int H, int L, int T, int D,
                        int C, const void* q, const void* k, const void* v,
                        const float* pos4, const float* weight, const float* bias,
                        const int32_t* lens, const float* lse, const void* grad_out,
                        const void* out, float scale, void* dq, void* dk, void* dv, float* dweight,
                        float* dbias, float* rowsum, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Longest event (in tokens) the kernels take for this dtype, flags and shape:
 * an event's rows of all heads -- q, k, v (three times D wide with
 * FST_QKV_INTERLEAVED) and the C-wide scratch of the backward -- must span
 * less than 2^31 bytes. Host-only, no GPU call. No reference counterpart
 * (the reference's Triton kernels state no bound). */
int fst_max_event_len(int dtype, int flags, int H, int D, int C);

/* The fp32 frequency ladder exp(-i ln(1e4) / (C/2)), i < C/2, that the kernels
 * embed with, written to out[0 .. C/2). Counterpart of sinusoidal_frequencies
 * (reference.py:45-56); evaluated with the same fp32 steps. */
void fst_frequencies(int C, float* out);

/* Message of the last failed call on this thread ("" if none). */
const char* fst_last_error(void);

/* Library version string, "flash-spacetime-gfx950 <major>.<minor>.<patch>
 * abi <n> build <id>", id a hash of the kernel sources. The abi number changes with every change of an entry point's
 * arguments or of what a caller must provide (workspace sizes are always
 * queried, so a larger workspace is not an ABI change): abi 2 added the
 * forward's output to fst_backward / fst_backward_phases (the argument
 * `out`, before `scale`). */
const char* fst_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FLASH_SPACETIME_H */
