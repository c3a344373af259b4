// gemm_tab_0.hip -- pxk_gemm kernel instantiations, part 1 of 6 of the (transpose, prologue,
// epilogue) table (the parts compile in parallel; gemm.hip searches them all).
#include "gemm_impl.hpp"

namespace pxk {
namespace gemm {

const Entry kTable0[] = {
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_NONE, PXK_EPI_STORE),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_NONE, PXK_EPI_MUL_X),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_NONE, PXK_EPI_ROPE_REL),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_NONE, PXK_EPI_ROPE_FWD),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_RMS, PXK_EPI_STORE),
};
const int kTable0Size = static_cast<int>(sizeof(kTable0) / sizeof(kTable0[0]));

}  // namespace gemm
}  // namespace pxk
