// Model exports and checkpoints into the device model (host code only).
//
// The reference's inference side loads weights with load_checkpoint(path, training =
// false) (src/train/checkpoint.cpp:186-324); the directory format is
// docs/file_formats.md ("Checkpoint directory"): manifest.json (format, version, the
// architecture and tokenizer hashes, parameter count, per-file SHA-256, one entry per
// tensor with name, role, shape, dtype, file, offset, byte count and CRC-32), COMPLETE
// (SHA-256 of the manifest text), config.json, tokenizer.json and weights.bin (f32 or
// f16 weights; a training checkpoint adds optimizer.bin and trainer_state.json).  This
// file checks a directory the same way, in the same order and with the same error
// codes and messages, converts the weights to fp32 in the registry order and hands them
// to mla_model_create / mla_engine_create.
//
// SHA-256, CRC-32 and the JSON reader are this library's own (mla_io.hpp); the reference
// uses CommonCrypto, its own CRC table and its own JSON class (src/core/io.cpp:111-150,
// src/core/json.cpp).
#include "mla_capi_util.hpp"
#include "mla_hip.h"
#include "mla_io.hpp"
#include "mla_tokenizer.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <set>
#include <stdexcept>
#include <string>
#include <utility>
#include <variant>
#include <vector>

namespace mla {
namespace {

using namespace io;

// ---------------------------------------------------- configuration ----
// ModelConfig::json().dump() (src/model/config.cpp:49-70): the architecture's identity.
std::string config_dump(const mla_model_config& c) {
    std::map<std::string, std::string> kv = {
        {"model_type", dump_string("mla_dense_decoder")},
        {"version", dump_number(1)},
        {"vocab_size", dump_number(c.vocab_size)},
        {"max_sequence_length", dump_number(c.max_sequence_length)},
        {"n_layers", dump_number(c.n_layers)},
        {"d_model", dump_number(c.d_model)},
        {"n_heads", dump_number(c.n_heads)},
        {"head_dim_nope", dump_number(c.head_dim_nope)},
        {"head_dim_rope", dump_number(c.head_dim_rope)},
        {"head_dim_value", dump_number(c.head_dim_value)},
        {"q_lora_rank", dump_number(c.q_lora_rank)},
        {"kv_lora_rank", dump_number(c.kv_lora_rank)},
        {"d_ff", dump_number(c.d_ff)},
        {"norm_epsilon", dump_number((double)c.norm_epsilon)},
        {"rope_theta", dump_number((double)c.rope_theta)},
        {"norm", dump_string("rmsnorm")},
        {"activation", dump_string("swiglu")},
        {"mla_latent_norms", "true"},
        {"bias", "false"},
        {"tie_word_embeddings", "true"}};
    std::string s = "{";
    for (const auto& [k, v] : kv) {
        if (s.size() > 1)
            s += ',';
        s += dump_string(k) + ':' + v;
    }
    return s + '}';
}

// ModelConfig::from_json (src/model/config.cpp:74-107): MLA_OK or the reference's code
// and message.
int config_from_json(const Json& j, mla_model_config& c) {
    try {
        c.vocab_size = j.at("vocab_size").integer();
        c.max_sequence_length = j.at("max_sequence_length").integer();
        c.n_layers = j.at("n_layers").integer();
        c.d_model = j.at("d_model").integer();
        c.n_heads = j.at("n_heads").integer();
        c.head_dim_nope = j.at("head_dim_nope").integer();
        c.head_dim_rope = j.at("head_dim_rope").integer();
        c.head_dim_value = j.at("head_dim_value").integer();
        c.q_lora_rank = j.at("q_lora_rank").integer();
        c.kv_lora_rank = j.at("kv_lora_rank").integer();
        c.d_ff = j.at("d_ff").integer();
        c.norm_epsilon = (float)j.at("norm_epsilon").number();
        c.rope_theta = (float)j.at("rope_theta").number();
        if (j.str_or("model_type", "mla_dense_decoder") != "mla_dense_decoder" ||
            j.num_or("version", 1) != 1 || j.str_or("norm", "rmsnorm") != "rmsnorm" ||
            j.str_or("activation", "swiglu") != "swiglu" || j.bool_or("bias", false) ||
            !j.bool_or("tie_word_embeddings", true) || !j.bool_or("mla_latent_norms", true))
            return fail(MLA_ERR_UNSUPPORTED,
                        "Only v1 tied-embedding, bias-free MLA with latent RMSNorm and SwiGLU "
                        "is supported");
        const int st = mla_config_validate(&c);
        if (st != MLA_OK)
            return st;
        if (j.contains("expected_parameter_count") &&
            j.at("expected_parameter_count").size_integer() != mla_config_parameter_count(&c))
            return fail(MLA_ERR_INVALID_ARGUMENT,
                        "Expected parameter count disagrees with architecture");
        return MLA_OK;
    } catch (const std::exception& e) {
        return fail(MLA_ERR_INVALID_ARGUMENT, e.what());
    }
}

int parse_file(const std::string& path, Json& out) {  // read_json
    std::string text, err;
    if (!read_file(path, text, err))
        return fail(MLA_ERR_IO, err);
    try {
        out = JsonReader(text).parse();
    } catch (const std::exception& e) {
        return fail(MLA_ERR_INVALID_ARGUMENT, e.what());
    }
    return MLA_OK;
}

int load_config(const std::string& path, mla_model_config& c) {  // ModelConfig::load
    Json j;
    const int st = parse_file(path, j);
    return st != MLA_OK ? st : config_from_json(j, c);
}

// ------------------------------------------------------------ tokenizer ----
// Tokenizer::load's checks (tokenizer.cpp:70-127); the tokenizer's identity is the
// SHA-256 of its file bytes.
int check_tokenizer(const std::string& path, int& vocab, std::string& hash) {
    Tokenizer t;
    const int st = tokenizer_load(path, t);
    if (st != MLA_OK)
        return st;
    vocab = t.vocab;
    hash = t.hash;
    return MLA_OK;
}

// ------------------------------------------------------------- registry ----
struct Slot {
    size_t offset, rows, cols;
    const char* role;
};

// Parameter names, roles and shapes in registry order (src/model/model.cpp:26-63).
std::map<std::string, Slot> registry(const mla_model_config& c) {
    static const char* names[13] = {"attn.norm",    "attn.w_dq", "attn.q_norm", "attn.w_uq",
                                    "attn.w_dkv",   "attn.kv_norm", "attn.w_uk", "attn.w_uv",
                                    "attn.w_o",     "ffn.norm",  "ffn.w_gate",  "ffn.w_up",
                                    "ffn.w_down"};
    static const char* roles[13] = {"norm_scale",    "hidden_matrix", "norm_scale",
                                    "hidden_matrix", "hidden_matrix", "norm_scale",
                                    "hidden_matrix", "hidden_matrix", "hidden_matrix",
                                    "norm_scale",    "hidden_matrix", "hidden_matrix",
                                    "hidden_matrix"};
    const size_t d = c.d_model, q = c.q_lora_rank, kv = c.kv_lora_rank, H = c.n_heads;
    const size_t nope = c.head_dim_nope, rope = c.head_dim_rope, dv = c.head_dim_value,
                 ff = c.d_ff;
    const size_t shapes[13][2] = {{1, d},         {d, q},       {1, q},         {q, H * (nope + rope)},
                                  {d, kv + rope}, {1, kv},      {kv, H * nope}, {kv, H * dv},
                                  {H * dv, d},    {1, d},       {d, ff},        {d, ff},
                                  {ff, d}};
    std::map<std::string, Slot> r;
    size_t at = 0;
    auto add = [&](const std::string& name, const char* role, size_t rows, size_t cols) {
        r.emplace(name, Slot{at, rows, cols, role});
        at += rows * cols;
    };
    add("token_embedding", "token_embedding", (size_t)c.vocab_size, d);
    add("final_norm", "norm_scale", 1, d);
    for (int l = 0; l < c.n_layers; ++l)
        for (int k = 0; k < 13; ++k)
            add("layers." + std::to_string(l) + "." + names[k], roles[k], shapes[k][0],
                shapes[k][1]);
    return r;
}

float half_to_float(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// load_checkpoint(path, training = false) (src/train/checkpoint.cpp:186-324).
int read_export(const std::string& dir, mla_model_config& cfg, float* params, size_t count) {
    std::string raw, err;
    if (!read_file(join(dir, "manifest.json"), raw, err))
        return fail(MLA_ERR_IO, err);
    std::string complete;
    if (!read_file(join(dir, "COMPLETE"), complete, err) || complete != sha256_hex(raw) + "\n")
        return fail(MLA_ERR_IO, "Checkpoint is incomplete or manifest checksum failed");
    Json manifest;
    try {
        manifest = JsonReader(raw).parse();
    } catch (const std::exception& e) {
        return fail(MLA_ERR_INVALID_ARGUMENT, e.what());
    }
    try {
        const std::string format = manifest.at("format").string();
        if ((format != "mini-mla-checkpoint" && format != "mini-mla-model") ||
            manifest.at("version").integer() != 1)
            return fail(MLA_ERR_UNSUPPORTED,
                        "Unsupported model format or inference export used for resume");
        int st = load_config(join(dir, "config.json"), cfg);
        if (st != MLA_OK)
            return st;
        const size_t n_params = mla_config_parameter_count(&cfg);
        if (sha256_hex(config_dump(cfg)) != manifest.at("model_config_sha256").string() ||
            n_params != manifest.at("parameter_count").size_integer())
            return fail(MLA_ERR_INVALID_ARGUMENT, "Checkpoint model configuration mismatch");
        int vocab = 0;
        std::string tok_hash;
        st = check_tokenizer(join(dir, "tokenizer.json"), vocab, tok_hash);
        if (st != MLA_OK)
            return st;
        if (tok_hash != manifest.at("tokenizer_sha256").string() || vocab != cfg.vocab_size)
            return fail(MLA_ERR_INVALID_ARGUMENT, "Checkpoint tokenizer mismatch");
        if (params && count != n_params)
            return fail(MLA_ERR_INVALID_ARGUMENT,
                        "parameter buffer holds " + std::to_string(count) +
                            " floats; the export has " + std::to_string(n_params));
        std::map<std::string, std::string> files;
        for (const auto& [name, hash] : manifest.at("sha256").object()) {
            if (name != "weights.bin" && name != "optimizer.bin" && name != "trainer_state.json")
                throw std::invalid_argument("Invalid checkpoint filename");
            std::string bytes;
            if (!read_file(join(dir, name.c_str()), bytes, err))
                return fail(MLA_ERR_IO, err);
            if (sha256_hex(bytes) != hash.string())
                throw std::invalid_argument("Checkpoint file checksum failed: " + name);
            files.emplace(name, std::move(bytes));
        }
        std::map<std::string, Slot> expected = registry(cfg);
        std::set<std::string> seen;
        std::map<std::string, size_t> ends;
        for (const Json& entry : manifest.at("tensors").array()) {
            const std::string name = entry.at("name").string(), file = entry.at("file").string(),
                              dtype = entry.at("dtype").string();
            if (file != "weights.bin" && file != "optimizer.bin")
                throw std::invalid_argument("Invalid tensor filename");
            if (!seen.insert(name).second)
                throw std::invalid_argument("Duplicate named tensor");
            const size_t offset = entry.at("offset").size_integer(),
                         nbytes = entry.at("nbytes").size_integer();
            auto fit = files.find(file);
            if (fit == files.end() || offset != ends[file] || offset > fit->second.size() ||
                nbytes > fit->second.size() - offset)
                throw std::invalid_argument("Invalid tensor extent or missing tensor file");
            const uint8_t* bytes = reinterpret_cast<const uint8_t*>(fit->second.data()) + offset;
            ends[file] = offset + nbytes;
            if (crc32(bytes, nbytes) != entry.at("crc32").size_integer())
                throw std::invalid_argument("Tensor checksum failed: " + name);
            auto it = expected.find(name);
            if (it == expected.end()) {
                if (file == "optimizer.bin" && format == "mini-mla-checkpoint")
                    continue;  // training state: not needed for inference
                throw std::invalid_argument("Unexpected tensor: " + name);
            }
            const Slot slot = it->second;
            const Json::Array& shape = entry.at("shape").array();
            const size_t item = dtype == "f32" ? 4 : dtype == "f16" ? 2 : 0;
            if (!item || file != "weights.bin" || shape.size() != 2 ||
                shape[0].integer() != (int)slot.rows || shape[1].integer() != (int)slot.cols ||
                nbytes != slot.rows * slot.cols * item || entry.at("role").string() != slot.role)
                throw std::invalid_argument("Tensor shape, dtype, role, or file mismatch: " +
                                            name);
            const size_t n = slot.rows * slot.cols;
            bool finite = true;
            for (size_t k = 0; k < n; ++k) {
                float x;
                if (item == 4) {
                    std::memcpy(&x, bytes + 4 * k, 4);
                } else {
                    uint16_t h;
                    std::memcpy(&h, bytes + 2 * k, 2);
                    x = half_to_float(h);
                }
                finite = finite && std::isfinite(x);
                if (params)
                    params[slot.offset + k] = x;
            }
            if (!finite)
                throw std::invalid_argument("Nonfinite checkpoint tensor: " + name);
            expected.erase(it);
        }
        if (!expected.empty())
            throw std::invalid_argument("Checkpoint is missing tensor: " + expected.begin()->first);
        for (const auto& [file, end] : ends)
            if (end != files.at(file).size())
                throw std::invalid_argument("Unindexed trailing tensor data");
        return MLA_OK;
    } catch (const std::exception& e) {
        return fail(MLA_ERR_IO, e.what());
    }
}

}  // namespace
}  // namespace mla

using namespace mla;

extern "C" {

int mla_export_read_config(const char* dir, mla_model_config* config) {
    if (!dir || !config)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_export_read_config: null argument");
    return load_config(join(dir, "config.json"), *config);
}

int mla_export_read(const char* dir, mla_model_config* config, float* params,
                    size_t params_count) {
    if (!dir || !config)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_export_read: null argument");
    return read_export(dir, *config, params, params_count);
}

int mla_config_hash(const mla_model_config* config, char* hex_out) {
    if (!config || !hex_out)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_config_hash: null argument");
    const std::string h = sha256_hex(config_dump(*config));
    std::memcpy(hex_out, h.c_str(), 65);
    return MLA_OK;
}

int mla_model_load(const char* dir, int max_batch, int page_size, mla_model_config* config,
                   void** model) {
    if (!dir || !config || !model)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_model_load: null argument");
    mla_model_config c{};
    int st = load_config(join(dir, "config.json"), c);
    if (st != MLA_OK)
        return st;
    std::vector<float> params(mla_config_parameter_count(&c));
    st = read_export(dir, c, params.data(), params.size());
    if (st != MLA_OK)
        return st;
    *config = c;
    return mla_model_create(&c, params.data(), max_batch, page_size, model);
}

int mla_engine_load(const char* dir, int max_sessions, int max_rows, int num_pages,
                    int page_size, mla_model_config* config, void** engine) {
    if (!dir || !config || !engine)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_engine_load: null argument");
    mla_model_config c{};
    int st = load_config(join(dir, "config.json"), c);
    if (st != MLA_OK)
        return st;
    std::vector<float> params(mla_config_parameter_count(&c));
    st = read_export(dir, c, params.data(), params.size());
    if (st != MLA_OK)
        return st;
    *config = c;
    return mla_engine_create(&c, params.data(), max_sessions, max_rows, num_pages, page_size,
                             engine);
}

}  // extern "C"
