/** @file checkpoint.hpp
 *  @brief Hugging Face checkpoints to the device: config.json (ParseHfConfig, src/hf_model.cpp:99-240),
 *         safetensors files, single or sharded (include/pulsatrix/safetensors.hpp; HfCheckpoint), and
 *         LoadCausalLM (src/causal_lm.cpp:293-301) with the weights converted on the GPU.
 *
 *  Each tensor's raw bytes are copied to HBM as stored (BF16 checkpoints move half the bytes of
 *  fp32) and widened / transposed there by pxk_convert_weight, straight into the module's
 *  parameter storage. Every mapping is checked (names, shapes, dtypes) before the first write, as
 *  LoadWeights does (src/causal_lm.cpp:179-255).
 */
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <string_view>
#include <vector>

#include "pulsatrix/causal_lm.hpp"
#include "pulsatrix/hf_model.hpp"

namespace pulsatrix {

/** @brief The subset of config.json the Llama-family path reads; throws std::invalid_argument
 *         (with the reference's "HfModelConfig: ..." wording) on malformed or unsupported input. */
HfModelConfig ParseHfConfig(std::string_view json);
HfModelConfig ReadHfConfig(const std::string& path);

/** @brief One tensor of a safetensors file. */
struct SafetensorsTensorInfo {
    std::string dtype;  // "F32", "BF16", ...
    std::vector<int64_t> shape;
    int64_t data_begin = 0, data_end = 0;  // byte offsets into the data section
};

/** @brief A memory-mapped safetensors file (8-byte little-endian header length, JSON header,
 *         data). Validated on open: offsets inside the data section, sizes matching shape x dtype. */
class SafetensorsFile {
public:
    static SafetensorsFile Map(const std::string& path);
    [[nodiscard]] bool contains(const std::string& name) const { return infos_.count(name) != 0; }
    [[nodiscard]] const SafetensorsTensorInfo& info(const std::string& name) const;
    [[nodiscard]] std::vector<std::string> names() const;
    /** @brief The raw bytes of `name`, valid while this object (or a copy) lives. */
    [[nodiscard]] std::pair<const uint8_t*, size_t> bytes(const std::string& name) const;

private:
    struct Mapping;
    std::shared_ptr<const Mapping> map_;
    int64_t data_start_ = 0;
    std::map<std::string, SafetensorsTensorInfo> infos_;
};

/** @brief A checkpoint directory: model.safetensors, or the shards model.safetensors.index.json names. */
class HfCheckpoint {
public:
    static HfCheckpoint Open(const std::string& directory);
    [[nodiscard]] bool contains(const std::string& name) const { return where_.count(name) != 0; }
    [[nodiscard]] const SafetensorsFile& file_of(const std::string& name) const;
    [[nodiscard]] std::vector<std::string> names() const;

private:
    std::vector<SafetensorsFile> files_;
    std::map<std::string, size_t> where_;
};

/** @brief config.json + weights of `directory` into a new CausalLM on `backend` (an MI355XBackend). */
std::unique_ptr<CausalLM> LoadCausalLM(const std::string& directory, DeviceBackend* backend);

}  // namespace pulsatrix
