// gemm_tab_4.hip -- pxk_gemm kernel instantiations, part 5 of 6 of the (transpose, prologue,
// epilogue) table (the parts compile in parallel; gemm.hip searches them all).
#include "gemm_impl.hpp"

namespace pxk {
namespace gemm {

const Entry kTable4[] = {
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_NONE, PXK_EPI_STORE_BIAS),
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_DIV_STAB, PXK_EPI_MUL_X),
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_DIV_STAB, PXK_EPI_SWIGLU_REL),
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_NONE, PXK_EPI_SPV),
};
const int kTable4Size = static_cast<int>(sizeof(kTable4) / sizeof(kTable4[0]));

}  // namespace gemm
}  // namespace pxk
