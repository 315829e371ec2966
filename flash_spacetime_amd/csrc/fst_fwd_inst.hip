// Instantiates the forward kernel for one (dtype, D) over every supported
// head padding HP in {4, 8, 12, 16} and channel count C in {16, 32, 48, 64}.
// Built once per (dtype, D) with -DFST_T=<bf16|float> -DFST_D=<D>
// -DFST_NAME=<dtype>_<D> so the instances compile in parallel.
#include "fst_forward.hip"
#include "fst_fwd2.hip"

#if !defined(FST_T) || !defined(FST_D) || !defined(FST_NAME)
#error "FST_T, FST_D and FST_NAME must be defined"
#endif

#define FST_CAT2(a, b) a##b
#define FST_CAT(a, b) FST_CAT2(a, b)

namespace fst {

int FST_CAT(fwd_dispatch_, FST_NAME)(const FwdParams& prm, int HP, int C, hipStream_t stream, int grid, bool query,
                                     int* rows) {
  // bf16 runs the 16-row-tile kernel (fst_fwd2.hip) wherever its LDS plan
  // fits; fp32 and the remaining shapes run fst_forward.hip. With query set
  // nothing is launched: the plan bits of prm.flags are checked and *rows
  // receives the rows per workgroup of the variant they name.
#define FST_CASE(HPV, CV)                                                       \
  if (HP == HPV && C == CV) {                                                   \
    if constexpr (is_bf16<FST_T>::value && Fwd2Pick<HPV, FST_D, CV>::OK) {      \
      *rows = 16;                                                               \
      return fwd2_launch_t<HPV, FST_D, CV>(prm, stream, grid, query);           \
    } else {                                                                    \
      return fwd_launch_t<FST_T, HPV, FST_D, CV>(prm, stream, grid, query, rows); \
    }                                                                           \
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

// FST_PLAN_FWD_* bits compiled for head padding HP and C channels.
int FST_CAT(fwd_plans_, FST_NAME)(int HP, int C) {
#define FST_CASE(HPV, CV)                                                   \
  if (HP == HPV && C == CV) {                                               \
    if constexpr (is_bf16<FST_T>::value && Fwd2Pick<HPV, FST_D, CV>::OK)    \
      return Fwd2Pick<HPV, FST_D, CV>::PLANS;                               \
    else                                                                    \
      return FwdPick<FST_T, HPV, FST_D, CV>::PLANS;                         \
  }
#define FST_CASES(HPV) FST_CASE(HPV, 16) FST_CASE(HPV, 32) FST_CASE(HPV, 48) FST_CASE(HPV, 64)
  FST_CASES(4)
  FST_CASES(8)
  FST_CASES(12)
  FST_CASES(16)
#undef FST_CASES
#undef FST_CASE
  return 0;
}

}  // namespace fst
