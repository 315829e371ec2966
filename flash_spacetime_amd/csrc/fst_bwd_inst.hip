// Instantiates the backward kernels for one (dtype, D) over every head
// padding HP in {4, 8, 12, 16} and channel count C in {16, 32, 48, 64}.
// Built once per (dtype, D) with -DFST_T, -DFST_D and -DFST_NAME; for bf16
// twice, with -DFST_BWD_PART=1 (the tile rows kernel, bwd2_rows_dispatch_*,
// built with the machine scheduler's max-ilp strategy) and =2 (everything
// else).
#include "fst_backward.hip"
#include "fst_bwd2.hip"

#if !defined(FST_T) || !defined(FST_D) || !defined(FST_NAME)
#error "FST_T, FST_D and FST_NAME must be defined"
#endif

#define FST_CAT2(a, b) a##b
#define FST_CAT(a, b) FST_CAT2(a, b)

namespace fst {

// The bf16 tile rows kernel of (HP, C): launched (or, with query, checked)
// from its own translation unit (FST_BWD_PART = 1).
int FST_CAT(bwd2_rows_dispatch_, FST_NAME)(const BwdParams& prm, int HP, int C, hipStream_t stream, int grid,
                                           bool query);

#if FST_BWD_PART == 1
int FST_CAT(bwd2_rows_dispatch_, FST_NAME)(const BwdParams& prm, int HP, int C, hipStream_t stream, int grid,
                                           bool query) {
#define FST_CASE(HPV, CV)                                                      \
  if (HP == HPV && C == CV) {                                                  \
    if constexpr (Bwd2Pick<HPV, FST_D, CV>::OK)                                \
      return bwd2_launch_t<HPV, FST_D, CV>(prm, 0, stream, grid, query);       \
    return FST_EUNSUPPORTED;                                                   \
  }
#define FST_CASES(HPV) FST_CASE(HPV, 16) FST_CASE(HPV, 32) FST_CASE(HPV, 48) FST_CASE(HPV, 64)
  FST_CASES(4)
  FST_CASES(8)
  FST_CASES(12)
  FST_CASES(16)
#undef FST_CASES
#undef FST_CASE
  return FST_EUNSUPPORTED;
}
#else

int FST_CAT(bwd_dispatch_, FST_NAME)(const BwdParams& prm, int which, int HP, int C, hipStream_t stream, int grid,
                                     bool query, int* rows) {
  // bf16 runs the 16-row / 16-key tile kernels (fst_bwd2.hip) wherever their
  // LDS plan fits; fp32 and the remaining shapes run fst_backward.hip. With
  // query set nothing is launched: the plan bits of prm.flags are checked and
  // *rows receives the rows (keys) per workgroup of the variant they name.
#define FST_CASE(HPV, CV)                                                      \
  if (HP == HPV && C == CV) {                                                  \
    if constexpr (is_bf16<FST_T>::value && Bwd2Pick<HPV, FST_D, CV>::OK) {     \
      *rows = 16;                                                              \
      if constexpr (FST_BWD_PART == 2) {                                       \
        if (which == 0) return FST_CAT(bwd2_rows_dispatch_, FST_NAME)(prm, HP, C, stream, grid, query); \
      }                                                                        \
      return bwd2_launch_t<HPV, FST_D, CV>(prm, which, stream, grid, query);   \
    } else {                                                                   \
      return bwd_launch_t<FST_T, HPV, FST_D, CV>(prm, which, stream, grid, query, rows); \
    }                                                                          \
  }
#define FST_CASES(HPV) FST_CASE(HPV, 16) FST_CASE(HPV, 32) FST_CASE(HPV, 48) FST_CASE(HPV, 64)
  FST_CASES(4)
  FST_CASES(8)
  FST_CASES(12)
  FST_CASES(16)
#undef FST_CASES
#undef FST_CASE
  if (query) *rows = 0;
  return FST_EUNSUPPORTED;
}

// FST_PLAN_ROWS_* / FST_PLAN_COLS_* / FST_PLAN_BWD_* bits compiled for head
// padding HP and C channels. The eight-wave, one-workgroup rows plan runs
// at HP rounded up to a multiple of 8.
template <int HP, int C>
static int bwd_plans_at() {
  if constexpr (is_bf16<FST_T>::value && Bwd2Pick<HP, FST_D, C>::OK) {
    using P = Bwd2Pick<HP, FST_D, C>;
    constexpr int HP8 = (HP + 7) / 8 * 8;
    int plans = P::COLS_PLANS | FST_PLAN_ROWS_KV_REG;
    if constexpr (P::ROWS_W4) plans |= FST_PLAN_ROWS_W4;
    if constexpr (Bwd2Pick<HP8, FST_D, C>::OK && Bwd2Pick<HP8, FST_D, C>::ROWS_W8) plans |= FST_PLAN_ROWS_W8;
    if constexpr (P::ROWS_W8X2) plans |= FST_PLAN_ROWS_W8X2;
    if constexpr (P::KL_W4 || P::KL_W8X2) plans |= FST_PLAN_ROWS_KV_LDS;
    return plans;
  } else {
    if constexpr (!BwdPick<BwdRowsCfg, FST_T, HP, FST_D, C>::OK ||
                  !BwdPick<BwdColsCfg, FST_T, HP, FST_D, C>::OK)
      return 0;
    else
      return bwd_split_plans<FST_T, HP, FST_D, C>();
  }
}

int FST_CAT(bwd_plans_, FST_NAME)(int HP, int C) {
#define FST_CASE(HPV, CV) \
  if (HP == HPV && C == CV) return bwd_plans_at<HPV, CV>();
#define FST_CASES(HPV) FST_CASE(HPV, 16) FST_CASE(HPV, 32) FST_CASE(HPV, 48) FST_CASE(HPV, 64)
  FST_CASES(4)
  FST_CASES(8)
  FST_CASES(12)
  FST_CASES(16)
#undef FST_CASES
#undef FST_CASE
  return 0;
}

#endif  // FST_BWD_PART

}  // namespace fst
