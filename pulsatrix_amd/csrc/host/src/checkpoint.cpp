// Hugging Face checkpoints to the device (pulsatrix/checkpoint.hpp).
#include "pulsatrix/checkpoint.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <optional>
#include <set>
#include <sstream>
#include <stdexcept>
#include <utility>

#include "pxk.h"

namespace pulsatrix {
namespace {

// ---- a small JSON reader (RFC 8259 values; numbers as double) ---------------------------------

struct Json {
    enum class T { Null, Bool, Number, String, Array, Object } t = T::Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    [[nodiscard]] const Json* find(const std::string& key) const {
        if (t != T::Object) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonReader {
public:
    explicit JsonReader(std::string_view s) : s_(s) {}

    Json document() {
        Json v = value(0);
        ws();
        if (i_ != s_.size()) fail("trailing characters");
        return v;
    }

private:
    [[noreturn]] void fail(const std::string& what) const {
        throw std::invalid_argument("JSON: " + what + " at offset " + std::to_string(i_));
    }
    void ws() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
    }
    bool eat(char c) {
        ws();
        if (i_ < s_.size() && s_[i_] == c) {
            ++i_;
            return true;
        }
        return false;
    }
    void expect(char c) {
        if (!eat(c)) fail(std::string("expected '") + c + "'");
    }
    bool word(const char* w) {
        const size_t n = std::strlen(w);
        if (s_.substr(i_, n) == w) {
            i_ += n;
            return true;
        }
        return false;
    }
    static void utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) {
            out += static_cast<char>(cp);
        } else if (cp < 0x800) {
            out += static_cast<char>(0xC0 | (cp >> 6));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += static_cast<char>(0xE0 | (cp >> 12));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            out += static_cast<char>(0xF0 | (cp >> 18));
            out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }
    uint32_t hex4() {
        if (i_ + 4 > s_.size()) fail("short \\u escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = s_[i_++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
            else fail("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        expect('"');
        std::string out;
        while (true) {
            if (i_ >= s_.size()) fail("unterminated string");
            const char c = s_[i_++];
            if (c == '"') break;
            if (static_cast<unsigned char>(c) < 0x20) fail("control character in string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (i_ >= s_.size()) fail("unterminated escape");
            const char e = s_[i_++];
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00) {  // a surrogate pair
                        if (!word("\\u")) fail("lone high surrogate");
                        const uint32_t lo = hex4();
                        if (lo < 0xDC00 || lo >= 0xE000) fail("bad low surrogate");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        fail("lone low surrogate");
                    }
                    utf8(out, cp);
                    break;
                }
                default: fail("bad escape");
            }
        }
        return out;
    }
    Json value(int depth) {
        if (depth > 64) fail("nesting too deep");
        ws();
        if (i_ >= s_.size()) fail("unexpected end");
        Json v;
        const char c = s_[i_];
        if (c == '{') {
            ++i_;
            v.t = Json::T::Object;
            if (eat('}')) return v;
            do {
                ws();
                std::string key = string();
                expect(':');
                v.obj.emplace_back(std::move(key), value(depth + 1));
            } while (eat(','));
            expect('}');
        } else if (c == '[') {
            ++i_;
            v.t = Json::T::Array;
            if (eat(']')) return v;
            do v.arr.push_back(value(depth + 1));
            while (eat(','));
            expect(']');
        } else if (c == '"') {
            v.t = Json::T::String;
            v.str = string();
        } else if (word("true")) {
            v.t = Json::T::Bool;
            v.b = true;
        } else if (word("false")) {
            v.t = Json::T::Bool;
        } else if (word("null")) {
            v.t = Json::T::Null;
        } else if (c == '-' || (c >= '0' && c <= '9')) {
            const size_t start = i_;
            while (i_ < s_.size() && std::strchr("+-0123456789.eE", s_[i_]) != nullptr) ++i_;
            const std::string text(s_.substr(start, i_ - start));
            char* end = nullptr;
            v.t = Json::T::Number;
            v.num = std::strtod(text.c_str(), &end);
            if (end != text.c_str() + text.size()) fail("bad number");
        } else {
            fail("unexpected character");
        }
        return v;
    }

    std::string_view s_;
    size_t i_ = 0;
};

std::string read_text(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

// ---- config.json (ParseHfConfig, src/hf_model.cpp:99-240, the Llama-family fields) --------------

[[noreturn]] void bad_config(const std::string& what) { throw std::invalid_argument("HfModelConfig: " + what); }

std::optional<double> opt_number(const Json& o, const char* key) {
    const Json* v = o.find(key);
    if (v == nullptr || v->t == Json::T::Null) return std::nullopt;
    if (v->t != Json::T::Number) bad_config(std::string(key) + " must be a number");
    return v->num;
}
std::optional<int64_t> opt_integer(const Json& o, const char* key) {
    const auto d = opt_number(o, key);
    if (!d) return std::nullopt;
    if (*d != std::floor(*d) || std::fabs(*d) > 9.0e15) bad_config(std::string(key) + " must be an integer");
    return static_cast<int64_t>(*d);
}
int64_t required_positive(const Json& o, const char* key) {
    const auto v = opt_integer(o, key);
    if (!v) bad_config(std::string("missing ") + key);
    if (*v <= 0) bad_config(std::string(key) + " must be positive");
    return *v;
}
std::optional<bool> opt_bool(const Json& o, const char* key) {
    const Json* v = o.find(key);
    if (v == nullptr || v->t == Json::T::Null) return std::nullopt;
    if (v->t != Json::T::Bool) bad_config(std::string(key) + " must be true or false");
    return v->b;
}
std::optional<std::string> opt_string(const Json& o, const char* key) {
    const Json* v = o.find(key);
    if (v == nullptr || v->t == Json::T::Null) return std::nullopt;
    if (v->t != Json::T::String) bad_config(std::string(key) + " must be a string");
    return v->str;
}

// ---- safetensors dtypes ----------------------------------------------------------------------

struct DtypeInfo {
    const char* name;
    int bytes;
    int pxk;  // -1: not a floating-point dtype the loader converts
};
const DtypeInfo kDtypes[] = {{"BOOL", 1, -1}, {"U8", 1, -1},  {"I8", 1, -1},  {"I16", 2, -1}, {"U16", 2, -1},
                             {"I32", 4, -1},  {"U32", 4, -1}, {"I64", 8, -1}, {"U64", 8, -1},
                             {"F8_E4M3", 1, PXK_DTYPE_F8_E4M3}, {"F8_E5M2", 1, PXK_DTYPE_F8_E5M2},
                             {"F16", 2, PXK_DTYPE_F16}, {"BF16", 2, PXK_DTYPE_BF16}, {"F32", 4, PXK_DTYPE_F32},
                             {"F64", 8, PXK_DTYPE_F64}};

const DtypeInfo* find_dtype(const std::string& name) {
    for (const DtypeInfo& d : kDtypes)
        if (name == d.name) return &d;
    return nullptr;
}

}  // namespace

HfModelConfig ParseHfConfig(std::string_view json) {
    Json root;
    try {
        root = JsonReader(json).document();
    } catch (const std::exception& e) {
        bad_config(std::string("not valid JSON: ") + e.what());
    }
    if (root.t != Json::T::Object) bad_config("must be a JSON object");
    HfModelConfig c;
    if (const Json* arch = root.find("architectures"); arch && arch->t == Json::T::Array && !arch->arr.empty() &&
                                                        arch->arr[0].t == Json::T::String)
        c.architecture = arch->arr[0].str;
    const Json* text = root.find("text_config");  // a multimodal model's language model
    if (text != nullptr && text->t != Json::T::Object) bad_config("text_config must be an object");
    const Json& t = text != nullptr ? *text : root;
    c.model_type = opt_string(t, "model_type").value_or(opt_string(root, "model_type").value_or(""));
    c.hidden_size = required_positive(t, "hidden_size");
    c.intermediate_size = required_positive(t, "intermediate_size");
    c.num_hidden_layers = required_positive(t, "num_hidden_layers");
    c.num_attention_heads = required_positive(t, "num_attention_heads");
    c.vocab_size = required_positive(t, "vocab_size");
    c.num_key_value_heads = opt_integer(t, "num_key_value_heads").value_or(c.num_attention_heads);
    if (c.num_key_value_heads <= 0 || c.num_attention_heads % c.num_key_value_heads != 0)
        bad_config("num_attention_heads must be a positive multiple of num_key_value_heads");
    if (const auto hd = opt_integer(t, "head_dim")) {
        if (*hd <= 0) bad_config("head_dim must be positive");
        c.head_dim = *hd;
    } else {
        if (c.hidden_size % c.num_attention_heads != 0) bad_config("hidden_size must be divisible by num_attention_heads");
        c.head_dim = c.hidden_size / c.num_attention_heads;
    }
    c.rms_norm_eps = static_cast<float>(opt_number(t, "rms_norm_eps").value_or(1e-6));
    const Json* rp = t.find("rope_parameters");
    if (rp != nullptr && rp->t != Json::T::Object) rp = nullptr;
    const Json* rp_full = rp != nullptr ? rp->find("full_attention") : nullptr;
    if (const auto theta = opt_number(t, "rope_theta")) {
        c.rope_theta = static_cast<float>(*theta);
    } else if (rp_full != nullptr && rp_full->t == Json::T::Object) {
        c.rope_theta = static_cast<float>(opt_number(*rp_full, "rope_theta").value_or(10000.0));
    } else if (rp != nullptr) {
        c.rope_theta = static_cast<float>(opt_number(*rp, "rope_theta").value_or(10000.0));
    }
    if (const auto local = opt_number(t, "rope_local_base_freq")) {
        c.rope_local_base_freq = static_cast<float>(*local);
    } else if (const Json* rs = rp != nullptr ? rp->find("sliding_attention") : nullptr;
               rs != nullptr && rs->t == Json::T::Object) {
        if (const auto theta = opt_number(*rs, "rope_theta")) c.rope_local_base_freq = static_cast<float>(*theta);
    }
    // RoPE scaling (RopeScaling, hf_model.cpp:67-87): rope_scaling, or rope_parameters (the
    // full-attention layers' entry when it is per layer type); "default" means none.
    const Json* scaling = t.find("rope_scaling");
    if (scaling == nullptr || scaling->t == Json::T::Null) scaling = rp;
    if (scaling != nullptr && scaling->t == Json::T::Object) {
        if (const Json* full = scaling->find("full_attention"); full != nullptr && full->t == Json::T::Object)
            scaling = full;
        HfRopeScaling r;
        r.type = opt_string(*scaling, "rope_type").value_or(opt_string(*scaling, "type").value_or("default"));
        if (r.type != "default") {
            r.factor = static_cast<float>(opt_number(*scaling, "factor").value_or(1.0));
            r.low_freq_factor = static_cast<float>(opt_number(*scaling, "low_freq_factor").value_or(1.0));
            r.high_freq_factor = static_cast<float>(opt_number(*scaling, "high_freq_factor").value_or(1.0));
            r.original_max_position_embeddings = opt_integer(*scaling, "original_max_position_embeddings").value_or(0);
            if (r.type != "linear" && r.type != "llama3")
                bad_config("rope_scaling \"" + r.type + "\" is not on the MI355X path");
            c.rope_scaling = r;
        }
    } else if (scaling != nullptr && scaling->t != Json::T::Null) {
        bad_config("rope_scaling must be an object");
    }
    c.tie_word_embeddings = opt_bool(t, "tie_word_embeddings").value_or(opt_bool(root, "tie_word_embeddings").value_or(true));
    const std::string& type = c.model_type;
    const bool qwen2 = type == "qwen2" || type == "qwen2_moe";
    const bool gemma3 = type == "gemma3" || type == "gemma3_text";
    const std::optional<bool> attention_bias = opt_bool(t, "attention_bias");
    c.qkv_bias = attention_bias.value_or(qwen2);
    c.out_bias = qwen2 ? false : attention_bias.value_or(false);
    c.mlp_bias = opt_bool(t, "mlp_bias").value_or(false);
    c.qk_norm = type == "qwen3" || type == "qwen3_moe" || gemma3 || type == "olmo2";
    c.hidden_act = opt_string(t, "hidden_act").value_or(opt_string(t, "hidden_activation").value_or("silu"));
    c.max_position_embeddings = opt_integer(t, "max_position_embeddings").value_or(0);
    if (c.hidden_act != "silu" && c.hidden_act != "gelu_pytorch_tanh" && c.hidden_act != "gelu_new")
        bad_config("hidden_act \"" + c.hidden_act + "\" is not on the MI355X path");
    if (opt_bool(t, "use_sliding_window").value_or(true)) c.sliding_window = opt_integer(t, "sliding_window");
    if (const auto qs = opt_number(t, "query_pre_attn_scalar")) c.query_pre_attn_scalar = static_cast<float>(*qs);
    if (const Json* lt = t.find("layer_types"); lt != nullptr && lt->t != Json::T::Null) {
        if (lt->t != Json::T::Array) bad_config("layer_types must be a list");
        for (const Json& v : lt->arr) {
            if (v.t != Json::T::String) bad_config("layer_types must hold strings");
            if (v.str != "full_attention" && v.str != "sliding_attention")
                bad_config("layer type \"" + v.str + "\" is not on the MI355X path");
            c.layer_types.push_back(v.str);
        }
        if (static_cast<int64_t>(c.layer_types.size()) != c.num_hidden_layers)
            bad_config("layer_types must name one type per layer");
    }
    // A window no sequence can exceed changes nothing (hf_model.cpp:206-213).
    if (c.sliding_window && c.max_position_embeddings > 0 && *c.sliding_window >= c.max_position_embeddings)
        c.sliding_window.reset();
    if (c.sliding_window && c.layer_types.empty() && type == "qwen2")
        bad_config("Qwen2's sliding window without layer_types (max_window_layers) is not on the MI355X path");
    if (gemma3) {  // (1 + w) RMSNorms, embeddings scaled by sqrt(hidden_size), sandwich norms (hf_model.cpp:221-228)
        c.norm_weight_offset = 1.0f;
        c.embed_scale = static_cast<float>(std::sqrt(static_cast<double>(c.hidden_size)));
        c.post_norms = true;
    } else if (type.rfind("gemma", 0) == 0) {
        bad_config("Gemma 1 and 2 (" + type + ") are not on the MI355X path");
    }
    for (const char* softcap : {"attn_logit_softcapping", "final_logit_softcapping"}) {
        const Json* v = t.find(softcap);
        if (v != nullptr && v->t != Json::T::Null)
            bad_config(std::string("logit softcapping (") + softcap + ") is not on the MI355X path");
    }
    return c;
}

HfModelConfig ReadHfConfig(const std::string& path) { return ParseHfConfig(read_text(path)); }

// ---- safetensors ------------------------------------------------------------------------------

struct SafetensorsFile::Mapping {
    const uint8_t* data = nullptr;
    size_t size = 0;
    ~Mapping() {
        if (data != nullptr && size > 0) munmap(const_cast<uint8_t*>(data), size);
    }
};

SafetensorsFile SafetensorsFile::Map(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) throw std::runtime_error("safetensors: cannot open " + path);
    struct stat st {};
    if (fstat(fd, &st) != 0 || st.st_size < 8) {
        ::close(fd);
        throw std::invalid_argument("safetensors: " + path + " is too short");
    }
    auto m = std::make_shared<Mapping>();
    m->size = static_cast<size_t>(st.st_size);
    void* p = mmap(nullptr, m->size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (p == MAP_FAILED) {
        m->size = 0;
        throw std::runtime_error("safetensors: cannot map " + path);
    }
    m->data = static_cast<const uint8_t*>(p);
    uint64_t hlen = 0;
    for (int b = 0; b < 8; ++b) hlen |= static_cast<uint64_t>(m->data[b]) << (8 * b);
    if (hlen > m->size - 8) throw std::invalid_argument("safetensors: header length past the end of " + path);
    Json header;
    try {
        header = JsonReader(std::string_view(reinterpret_cast<const char*>(m->data) + 8, hlen)).document();
    } catch (const std::exception& e) {
        throw std::invalid_argument(std::string("safetensors: bad header: ") + e.what());
    }
    if (header.t != Json::T::Object) throw std::invalid_argument("safetensors: header must be an object");
    SafetensorsFile f;
    f.map_ = m;
    f.data_start_ = static_cast<int64_t>(8 + hlen);
    const int64_t data_size = static_cast<int64_t>(m->size) - f.data_start_;
    for (const auto& [name, v] : header.obj) {
        if (name == "__metadata__") continue;
        const Json* dt = v.find("dtype");
        const Json* shape = v.find("shape");
        const Json* offs = v.find("data_offsets");
        if (!dt || dt->t != Json::T::String || !shape || shape->t != Json::T::Array || !offs ||
            offs->t != Json::T::Array || offs->arr.size() != 2)
            throw std::invalid_argument("safetensors: bad entry for \"" + name + "\"");
        const DtypeInfo* di = find_dtype(dt->str);
        if (di == nullptr) throw std::invalid_argument("safetensors: unknown dtype " + dt->str);
        SafetensorsTensorInfo info;
        info.dtype = dt->str;
        int64_t count = 1;
        for (const Json& d : shape->arr) {
            if (d.t != Json::T::Number || d.num < 0 || d.num != std::floor(d.num) || d.num > 9.0e15)
                throw std::invalid_argument("safetensors: bad shape for \"" + name + "\"");
            info.shape.push_back(static_cast<int64_t>(d.num));
            count *= info.shape.back();
        }
        for (const Json& o : offs->arr)
            if (o.t != Json::T::Number || o.num < 0 || o.num != std::floor(o.num))
                throw std::invalid_argument("safetensors: bad data_offsets for \"" + name + "\"");
        info.data_begin = static_cast<int64_t>(offs->arr[0].num);
        info.data_end = static_cast<int64_t>(offs->arr[1].num);
        if (info.data_end < info.data_begin || info.data_end > data_size)
            throw std::invalid_argument("safetensors: \"" + name + "\" lies outside the data section");
        if (info.data_end - info.data_begin != count * di->bytes)
            throw std::invalid_argument("safetensors: \"" + name + "\" has the wrong byte size for its shape");
        f.infos_.emplace(name, std::move(info));
    }
    return f;
}

const SafetensorsTensorInfo& SafetensorsFile::info(const std::string& name) const {
    const auto it = infos_.find(name);
    if (it == infos_.end()) throw std::invalid_argument("safetensors: no tensor \"" + name + "\"");
    return it->second;
}

std::vector<std::string> SafetensorsFile::names() const {
    std::vector<std::string> out;
    for (const auto& kv : infos_) out.push_back(kv.first);
    return out;
}

std::pair<const uint8_t*, size_t> SafetensorsFile::bytes(const std::string& name) const {
    const SafetensorsTensorInfo& i = info(name);
    return {map_->data + data_start_ + i.data_begin, static_cast<size_t>(i.data_end - i.data_begin)};
}

HfCheckpoint HfCheckpoint::Open(const std::string& directory) {
    namespace fs = std::filesystem;
    HfCheckpoint c;
    const fs::path dir(directory);
    const fs::path index = dir / "model.safetensors.index.json";
    std::vector<std::string> files;
    if (fs::exists(index)) {
        const Json j = JsonReader(read_text(index.string())).document();
        const Json* map = j.find("weight_map");
        if (map == nullptr || map->t != Json::T::Object)
            throw std::invalid_argument("HfCheckpoint: " + index.string() + " has no weight_map");
        std::set<std::string> seen;
        for (const auto& [name, file] : map->obj) {
            if (file.t != Json::T::String) throw std::invalid_argument("HfCheckpoint: bad weight_map entry");
            if (seen.insert(file.str).second) files.push_back(file.str);
        }
    } else if (fs::exists(dir / "model.safetensors")) {
        files.push_back("model.safetensors");
    } else {
        throw std::invalid_argument("HfCheckpoint: no model.safetensors or model.safetensors.index.json in " + directory);
    }
    for (const std::string& f : files) {
        c.files_.push_back(SafetensorsFile::Map((dir / f).string()));
        for (const std::string& name : c.files_.back().names()) {
            if (!c.where_.emplace(name, c.files_.size() - 1).second)
                throw std::invalid_argument("HfCheckpoint: tensor \"" + name + "\" appears in two files");
        }
    }
    return c;
}

const SafetensorsFile& HfCheckpoint::file_of(const std::string& name) const {
    const auto it = where_.find(name);
    if (it == where_.end()) throw std::invalid_argument("HfCheckpoint: no tensor \"" + name + "\"");
    return files_[it->second];
}

std::vector<std::string> HfCheckpoint::names() const {
    std::vector<std::string> out;
    for (const auto& kv : where_) out.push_back(kv.first);
    return out;
}

// ---- LoadCausalLM ------------------------------------------------------------------------------

std::unique_ptr<CausalLM> LoadCausalLM(const std::string& directory, DeviceBackend* backend) {
    auto* be = detail::require_mi355x(backend, "LoadCausalLM");
    const HfModelConfig config = ReadHfConfig((std::filesystem::path(directory) / "config.json").string());
    auto model = std::make_unique<CausalLM>(config, backend);
    const HfCheckpoint ckpt = HfCheckpoint::Open(directory);

    // The Hugging Face names and transforms of HuggingFaceMapping (src/causal_lm.cpp:257-291).
    struct Target {
        std::string source;
        Tensor* tensor;
        bool transpose;
    };
    std::vector<Target> targets;
    targets.push_back({"model.embed_tokens.weight", &model->embed_tokens().weight(), false});
    targets.push_back({"model.norm.weight", &model->norm().gamma(), false});
    for (int64_t i = 0; i < model->num_layers(); ++i) {
        const std::string hf = "model.layers." + std::to_string(i) + ".";
        TransformerBlock& blk = model->layer(i);
        targets.push_back({hf + "input_layernorm.weight", &blk.norm1().gamma(), false});
        if (config.post_norms) {  // Gemma 3: the sandwich norms and the MLP's pre-norm
            targets.push_back({hf + "post_attention_layernorm.weight", &blk.post_attn_norm().gamma(), false});
            targets.push_back({hf + "pre_feedforward_layernorm.weight", &blk.norm2().gamma(), false});
            targets.push_back({hf + "post_feedforward_layernorm.weight", &blk.post_mlp_norm().gamma(), false});
        } else {
            targets.push_back({hf + "post_attention_layernorm.weight", &blk.norm2().gamma(), false});
        }
        MultiHeadAttentionModule& mha = blk.mha();
        if (config.qk_norm) {
            targets.push_back({hf + "self_attn.q_norm.weight", &mha.q_norm().gamma(), false});
            targets.push_back({hf + "self_attn.k_norm.weight", &mha.k_norm().gamma(), false});
        }
        LinearModule* proj[] = {&mha.q_proj(), &mha.k_proj(), &mha.v_proj()};
        const char* names[] = {"q_proj", "k_proj", "v_proj"};
        for (int p = 0; p < 3; ++p) {
            targets.push_back({hf + "self_attn." + names[p] + ".weight", &proj[p]->weight(), true});
            if (config.qkv_bias) targets.push_back({hf + "self_attn." + names[p] + ".bias", &proj[p]->bias(), false});
        }
        targets.push_back({hf + "self_attn.o_proj.weight", &mha.out_proj().weight(), true});
        if (config.out_bias) targets.push_back({hf + "self_attn.o_proj.bias", &mha.out_proj().bias(), false});
        SwiGLUModule& mlp = blk.swiglu();
        LinearModule* mproj[] = {&mlp.gate_proj(), &mlp.up_proj(), &mlp.down_proj()};
        const char* mnames[] = {"gate_proj", "up_proj", "down_proj"};
        for (int p = 0; p < 3; ++p) {
            targets.push_back({hf + "mlp." + mnames[p] + ".weight", &mproj[p]->weight(), true});
            if (config.mlp_bias) targets.push_back({hf + "mlp." + mnames[p] + ".bias", &mproj[p]->bias(), false});
        }
    }
    if (!config.tie_word_embeddings) targets.push_back({"lm_head.weight", &model->lm_head()->weight(), true});

    // Check every mapping before the first write (LoadWeights, src/causal_lm.cpp:179-255).
    std::set<std::string> used;
    size_t staging = 0;
    for (const Target& t : targets) {
        if (!ckpt.contains(t.source))
            throw std::invalid_argument("LoadWeights: the checkpoint has no tensor \"" + t.source + "\"");
        const SafetensorsTensorInfo& info = ckpt.file_of(t.source).info(t.source);
        const DtypeInfo* di = find_dtype(info.dtype);
        if (di->pxk < 0)
            throw std::invalid_argument("safetensors: tensor \"" + t.source +
                                        "\" is an integer or bool tensor; only floating-point dtypes convert to a Tensor");
        std::vector<int64_t> dims = info.shape;
        if (t.transpose) {
            if (dims.size() != 2) throw std::invalid_argument("LoadWeights: \"" + t.source + "\" is not a matrix");
            std::swap(dims[0], dims[1]);
        }
        if (Shape(dims) != t.tensor->shape())
            throw std::invalid_argument("LoadWeights: \"" + t.source + "\" doesn't fit its target's shape");
        used.insert(t.source);
        staging = std::max(staging, static_cast<size_t>(info.data_end - info.data_begin));
    }
    for (const std::string& name : ckpt.names()) {  // strict, except a tied model's copy of the embedding
        if (used.count(name) || (config.tie_word_embeddings && name == "lm_head.weight")) continue;
        throw std::invalid_argument("LoadWeights: strict load failed: checkpoint tensor \"" + name + "\" unused");
    }

    // Raw bytes to HBM, then widened / transposed on the device into each parameter.
    Tensor stage = Tensor::uninitialized(Shape({static_cast<int64_t>((staging + 3) / 4)}), backend);
    for (const Target& t : targets) {
        const SafetensorsFile& f = ckpt.file_of(t.source);
        const SafetensorsTensorInfo& info = f.info(t.source);
        const auto [ptr, size] = f.bytes(t.source);
        be->copy(stage.data(), ptr, size, CopyDirection::HostToDevice);
        const int64_t rows = info.shape.size() == 2 ? info.shape[0] : 1;
        const int64_t cols = info.shape.size() == 2 ? info.shape[1] : t.tensor->numel();
        MI355XBackend::check(pxk_convert_weight(stage.data(), find_dtype(info.dtype)->pxk, rows, cols,
                                                t.transpose ? 1 : 0, t.tensor->data(), be->stream()),
                             "LoadCausalLM");
    }
    be->synchronize();
    return model;
}

}  // namespace pulsatrix
