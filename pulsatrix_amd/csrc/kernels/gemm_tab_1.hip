// gemm_tab_1.hip -- pxk_gemm kernel instantiations, part 2 of 6 of the (transpose, prologue,
// epilogue) table (the parts compile in parallel; gemm.hip searches them all).
#include "gemm_impl.hpp"

namespace pxk {
namespace gemm {

const Entry kTable1[] = {
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_NONE, PXK_EPI_STORE),
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_NONE, PXK_EPI_MUL_X),
    PXK_GEMM_ENTRY(1, 0, PXK_PRO_NONE, PXK_EPI_ROPE_REL),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_NONE, PXK_EPI_SWIGLU_FWD),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_RMS, PXK_EPI_STORE_BIAS),
};
const int kTable1Size = static_cast<int>(sizeof(kTable1) / sizeof(kTable1[0]));

}  // namespace gemm
}  // namespace pxk
