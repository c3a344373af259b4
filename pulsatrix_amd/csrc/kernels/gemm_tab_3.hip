// gemm_tab_3.hip -- pxk_gemm kernel instantiations, part 4 of 6 of the (transpose, prologue,
// epilogue) table (the parts compile in parallel; gemm.hip searches them all).
#include "gemm_impl.hpp"

namespace pxk {
namespace gemm {

const Entry kTable3[] = {
    PXK_GEMM_ENTRY(1, 1, PXK_PRO_NONE, PXK_EPI_STORE),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_DIV_STAB, PXK_EPI_MUL_X),
    PXK_GEMM_ENTRY(1, 0, PXK_PRO_NONE, PXK_EPI_VALUE_REL),
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_DIV_STAB, PXK_EPI_MUL_X_SPLIT),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_RMS, PXK_EPI_SWIGLU_FWD),
};
const int kTable3Size = static_cast<int>(sizeof(kTable3) / sizeof(kTable3[0]));

}  // namespace gemm
}  // namespace pxk
