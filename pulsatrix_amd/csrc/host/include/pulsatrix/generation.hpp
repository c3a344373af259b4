/** @file generation.hpp
 *  @brief The model as generation sees it (include/pulsatrix/generation.hpp:24): the token sequence
 *         so far in, the next token's logits out, one per vocabulary entry. The reference's
 *         Generate() drives any such function; CausalLM::next_token_logits() makes one over the
 *         MI355X decode kernels.
 */
#pragma once

#include <cstdint>
#include <functional>
#include <vector>

namespace pulsatrix {

using NextTokenLogitsFn = std::function<std::vector<float>(const std::vector<int64_t>& tokens)>;

}  // namespace pulsatrix
