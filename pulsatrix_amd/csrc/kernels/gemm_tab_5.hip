// gemm_tab_5.hip -- pxk_gemm kernel instantiations, part 6 of 6 of the (transpose, prologue,
// epilogue) table (the parts compile in parallel; gemm.hip searches them all).
#include "gemm_impl.hpp"

namespace pxk {
namespace gemm {

const Entry kTable5[] = {
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_NONE, PXK_EPI_ADD_RESID),
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_DIV_STAB, PXK_EPI_SPV),
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_NONE, PXK_EPI_MUL_X_SPLIT),
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_NONE, PXK_EPI_SWIGLU_REL),
};
const int kTable5Size = static_cast<int>(sizeof(kTable5) / sizeof(kTable5[0]));

}  // namespace gemm
}  // namespace pxk
