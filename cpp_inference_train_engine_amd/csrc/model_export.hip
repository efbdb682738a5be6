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

// ------------------------------------------------------------ validator ----
// A directory check is a pipeline of stages over one ExportScan; each stage either
// passes or names the failure (the reference's ErrorCode and message,
// load_checkpoint(path, training = false), src/train/checkpoint.cpp:186-324).  The stage
// order, and the rule order within a tensor entry, are the ones the failure-mode tests
// pin: a defect is reported by the first rule it breaks.
struct Failure {
    int code = MLA_OK;
    std::string message;
    explicit operator bool() const { return code != MLA_OK; }
};
Failure io_failure(std::string m) { return {MLA_ERR_IO, std::move(m)}; }

// One manifest tensor entry, as read from the manifest.
struct TensorEntry {
    std::string name, file, dtype, role;
    size_t offset = 0, nbytes = 0;
    uint32_t crc = 0;
    std::vector<long long> shape;
};

struct ExportScan {
    std::string dir;
    std::string manifest_text;
    Json manifest;
    bool training = false;  // a mini-mla-checkpoint (optimizer state may follow the weights)
    mla_model_config cfg{};
    size_t n_params = 0;
    std::map<std::string, std::string> files;      // every listed file, hash-verified
    std::map<std::string, size_t> cursor;          // next free byte of each tensor file
    std::map<std::string, Slot> pending;           // registry tensors not yet seen
    std::set<std::string> names;                   // entry names seen so far
    float* params = nullptr;                       // may be null: checks only
    size_t params_count = 0;
};

Failure seal_stage(ExportScan& x) {  // COMPLETE holds the manifest's SHA-256
    std::string err, complete;
    if (!read_file(join(x.dir, "manifest.json"), x.manifest_text, err))
        return io_failure(err);
    if (!read_file(join(x.dir, "COMPLETE"), complete, err) ||
        complete != sha256_hex(x.manifest_text) + "\n")
        return io_failure("Checkpoint is incomplete or manifest checksum failed");
    try {
        x.manifest = JsonReader(x.manifest_text).parse();
    } catch (const std::exception& e) {
        return {MLA_ERR_INVALID_ARGUMENT, e.what()};
    }
    return {};
}

Failure header_stage(ExportScan& x) {  // an inference export or a training checkpoint, v1
    const std::string format = x.manifest.at("format").string();
    x.training = format == "mini-mla-checkpoint";
    if ((!x.training && format != "mini-mla-model") || x.manifest.at("version").integer() != 1)
        return {MLA_ERR_UNSUPPORTED, "Unsupported model format or inference export used for resume"};
    return {};
}

Failure architecture_stage(ExportScan& x) {  // config.json is the manifest's architecture
    if (int st = load_config(join(x.dir, "config.json"), x.cfg))
        return {st, mla_last_error()};
    x.n_params = mla_config_parameter_count(&x.cfg);
    if (sha256_hex(config_dump(x.cfg)) != x.manifest.at("model_config_sha256").string() ||
        x.n_params != x.manifest.at("parameter_count").size_integer())
        return {MLA_ERR_INVALID_ARGUMENT, "Checkpoint model configuration mismatch"};
    return {};
}

Failure tokenizer_stage(ExportScan& x) {  // tokenizer.json is the manifest's, for this vocab
    Tokenizer tok;
    if (int st = tokenizer_load(join(x.dir, "tokenizer.json"), tok))
        return {st, mla_last_error()};
    if (tok.hash != x.manifest.at("tokenizer_sha256").string() || tok.vocab != x.cfg.vocab_size)
        return {MLA_ERR_INVALID_ARGUMENT, "Checkpoint tokenizer mismatch"};
    return {};
}

Failure files_stage(ExportScan& x) {  // every listed file exists and has its SHA-256
    static const std::set<std::string> kKnown = {"weights.bin", "optimizer.bin",
                                                 "trainer_state.json"};
    for (const auto& [file, digest] : x.manifest.at("sha256").object()) {
        if (!kKnown.count(file))
            return io_failure("Invalid checkpoint filename");
        std::string bytes, err;
        if (!read_file(join(x.dir, file.c_str()), bytes, err))
            return io_failure(err);
        if (sha256_hex(bytes) != digest.string())
            return io_failure("Checkpoint file checksum failed: " + file);
        x.files[file] = std::move(bytes);
    }
    x.pending = registry(x.cfg);
    return {};
}

TensorEntry read_entry(const Json& e) {
    TensorEntry t;
    t.name = e.at("name").string();
    t.file = e.at("file").string();
    t.dtype = e.at("dtype").string();
    t.role = e.at("role").string();
    t.offset = e.at("offset").size_integer();
    t.nbytes = e.at("nbytes").size_integer();
    t.crc = (uint32_t)e.at("crc32").size_integer();
    for (const Json& d : e.at("shape").array())
        t.shape.push_back(d.integer());
    return t;
}

size_t dtype_bytes(const std::string& dtype) { return dtype == "f32" ? 4 : dtype == "f16" ? 2 : 0; }

const uint8_t* entry_bytes(const ExportScan& x, const TensorEntry& t) {
    return reinterpret_cast<const uint8_t*>(x.files.at(t.file).data()) + t.offset;
}

// Widens the entry's values to fp32 (into params when given); false if one is not finite.
bool widen(const ExportScan& x, const TensorEntry& t, const Slot& slot) {
    const uint8_t* src = entry_bytes(x, t);
    const size_t n = slot.rows * slot.cols;
    bool finite = true;
    for (size_t k = 0; k < n; ++k) {
        float v;
        if (t.dtype == "f32") {
            std::memcpy(&v, src + 4 * k, 4);
        } else {
            uint16_t h;
            std::memcpy(&h, src + 2 * k, 2);
            v = half_to_float(h);
        }
        finite = finite && std::isfinite(v);
        if (x.params)
            x.params[slot.offset + k] = v;
    }
    return finite;
}

// What one manifest entry must satisfy, in the order the failure-mode tests pin.  A rule
// returns true when the entry passes it; `named` rules append the tensor's name.
enum class Verdict { pass, fail, skip };
struct EntryRule {
    const char* message;
    bool named;
    Verdict (*check)(ExportScan&, const TensorEntry&);
};
const EntryRule kEntryRules[] = {
    {"Invalid tensor filename", false,
     [](ExportScan&, const TensorEntry& t) {
         return t.file == "weights.bin" || t.file == "optimizer.bin" ? Verdict::pass : Verdict::fail;
     }},
    {"Duplicate named tensor", false,
     [](ExportScan& x, const TensorEntry& t) {
         return x.names.insert(t.name).second ? Verdict::pass : Verdict::fail;
     }},
    {"Invalid tensor extent or missing tensor file", false,
     [](ExportScan& x, const TensorEntry& t) {  // packed back to back, inside the file
         const auto f = x.files.find(t.file);
         if (f == x.files.end())
             return Verdict::fail;
         size_t& next = x.cursor[t.file];
         const size_t size = f->second.size();
         if (t.offset != next || t.offset > size || t.nbytes > size - t.offset)
             return Verdict::fail;
         next = t.offset + t.nbytes;
         return Verdict::pass;
     }},
    {"Tensor checksum failed: ", true,
     [](ExportScan& x, const TensorEntry& t) {
         return crc32(entry_bytes(x, t), t.nbytes) == t.crc ? Verdict::pass : Verdict::fail;
     }},
    {"Unexpected tensor: ", true,
     [](ExportScan& x, const TensorEntry& t) {
         if (x.pending.count(t.name))
             return Verdict::pass;
         // a training checkpoint's optimizer moments: not needed for inference
         return x.training && t.file == "optimizer.bin" ? Verdict::skip : Verdict::fail;
     }},
    {"Tensor shape, dtype, role, or file mismatch: ", true,
     [](ExportScan& x, const TensorEntry& t) {
         const Slot& s = x.pending.at(t.name);
         const size_t item = dtype_bytes(t.dtype);
         const bool ok = item && t.file == "weights.bin" && t.role == s.role &&
                         t.shape.size() == 2 && t.shape[0] == (long long)s.rows &&
                         t.shape[1] == (long long)s.cols && t.nbytes == s.rows * s.cols * item;
         return ok ? Verdict::pass : Verdict::fail;
     }},
    {"Nonfinite checkpoint tensor: ", true,
     [](ExportScan& x, const TensorEntry& t) {
         const auto it = x.pending.find(t.name);
         const bool finite = widen(x, t, it->second);
         x.pending.erase(it);
         return finite ? Verdict::pass : Verdict::fail;
     }},
};

Failure tensors_stage(ExportScan& x) {
    if (x.params && x.n_params != x.params_count)
        return {MLA_ERR_INVALID_ARGUMENT, "parameter buffer holds " +
                                              std::to_string(x.params_count) +
                                              " floats; the export has " +
                                              std::to_string(x.n_params)};
    for (const Json& raw : x.manifest.at("tensors").array()) {
        const TensorEntry t = read_entry(raw);
        for (const EntryRule& rule : kEntryRules) {
            const Verdict v = rule.check(x, t);
            if (v == Verdict::fail)
                return io_failure(rule.named ? rule.message + t.name : std::string(rule.message));
            if (v == Verdict::skip)
                break;
        }
    }
    return {};
}

Failure coverage_stage(ExportScan& x) {  // nothing missing, nothing unindexed
    if (!x.pending.empty())  // the first absent tensor in name order
        return io_failure("Checkpoint is missing tensor: " + x.pending.begin()->first);
    for (const auto& [file, end] : x.cursor)
        if (end != x.files.at(file).size())
            return io_failure("Unindexed trailing tensor data");
    return {};
}

// Reads a model export or checkpoint directory: every check of load_checkpoint(path,
// false) with its code and message; on success cfg is the architecture and params (when
// not null) holds count = parameter_count fp32 values in registry order.
int read_export(const std::string& dir, mla_model_config& cfg, float* params, size_t count) {
    ExportScan x;
    x.dir = dir;
    x.params = params;
    x.params_count = count;
    using Stage = Failure (*)(ExportScan&);
    static const Stage kStages[] = {seal_stage,  header_stage,   architecture_stage,
                                    tokenizer_stage, files_stage, tensors_stage,
                                    coverage_stage};
    for (size_t k = 0; k < sizeof(kStages) / sizeof(kStages[0]); ++k) {
        Failure f;
        try {
            f = kStages[k](x);
        } catch (const std::exception& e) {  // a manifest field missing or of the wrong type
            f = k == 0 ? Failure{MLA_ERR_INVALID_ARGUMENT, e.what()} : io_failure(e.what());
        }
        if (f)
            return fail(f.code, f.message);
    }
    cfg = x.cfg;
    return MLA_OK;
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
