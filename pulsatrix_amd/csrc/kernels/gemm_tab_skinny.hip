// gemm_tab_skinny.hip -- the skinny-M kernels of pxk_gemm (decode steps, last-row heads).
#include "gemm_impl.hpp"

namespace pxk {
namespace gemm {

const SkinnyEntry kSkinny[] = {
    PXK_SKINNY_NN(PXK_EPI_STORE),
    PXK_SKINNY_NN(PXK_EPI_STORE_BIAS),
    PXK_SKINNY_NN(PXK_EPI_ADD_RESID),
    PXK_SKINNY_NN(PXK_EPI_SWIGLU_FWD),
    SkinnyEntry{1,
                PXK_EPI_STORE,
                {{skinny_nt_kernel<4, PXK_EPI_STORE>}, {skinny_nt_kernel<8, PXK_EPI_STORE>}, {skinny_nt_kernel<16, PXK_EPI_STORE>}},
                {nullptr, nullptr, nullptr}},
};
const int kSkinnySize = static_cast<int>(sizeof(kSkinny) / sizeof(kSkinny[0]));

}  // namespace gemm
}  // namespace pxk
