// GGUF models, the tokenizer and text generation for the HIP path: the public
// model / context / generate entry points of tinyengine.h (reference
// c/src/tinyengine.c:270-372, c/src/gguf.c, c/src/tokenizer.c, c/src/ops.c:88-269,
// c/src/qwen.c:260-420, :1180-1250, :2489-2529).
//
// Host side (this file): the GGUF file is memory-mapped and parsed (header,
// metadata, tensor table, tokenizer arrays); tokenize / detokenize are the
// reference's byte-level BPE (GPT-2 byte alphabet, merges applied lowest rank
// first, special tokens matched longest-first at '<').  Device side: on the
// first GPU use the whole file is copied to HBM once; dequantize-row and
// matvec run there, and generation runs one token at a time through
// te_hip_decode_all_layers_f16 (every layer, then the head) with the embedding
// lookup, RoPE tables, fp16 KV cache and gathered norm / bias arrays in HBM.
// Greedy decoding takes the fused head + argmax; temperature sampling runs the
// head, keeps the logits that can enter the reference's top-k list on the
// device and draws on the host (te_hip_sample_top_k_f32).
#include "te_hip_common.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

// GGUF metadata value types (GGUF v2 / v3)
enum : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7, kStr = 8, kArr = 9,
    kU64 = 10, kI64 = 11, kF64 = 12
};

constexpr uint64_t kMaxCount = 1u << 20;  // metadata entries / tensors accepted (gguf.c:15)
constexpr uint64_t kMaxName = 4096;       // key / tensor-name bytes accepted (gguf.c:16)
constexpr uint64_t kMaxString = UINT64_MAX;

struct TypeInfo {
    uint32_t ggml;
    te_quant_kind quant;
    uint32_t block_elems, block_bytes;
};

// GGML tensor types as the reference's model info reports them (gguf.c:58-79).
constexpr TypeInfo kTypes[] = {
    {0, TE_QUANT_F32, 1, 4},           {1, TE_QUANT_F16, 1, 2},          {2, TE_QUANT_GGUF_Q4_0, 32, 18},
    {3, TE_QUANT_GGUF_Q4_1, 32, 20},   {6, TE_QUANT_GGUF_Q5_0, 32, 22},  {7, TE_QUANT_GGUF_Q5_1, 32, 24},
    {8, TE_QUANT_GGUF_Q8_0, 32, 34},   {10, TE_QUANT_GGUF_Q2_K, 256, 84}, {11, TE_QUANT_GGUF_Q3_K, 256, 110},
    {12, TE_QUANT_GGUF_Q4_K, 256, 144}, {13, TE_QUANT_GGUF_Q5_K, 256, 176}, {14, TE_QUANT_GGUF_Q6_K, 256, 210},
    {15, TE_QUANT_GGUF_Q8_K, 256, 292}, {16, TE_QUANT_GGUF_IQ2_XXS, 256, 66},
    {17, TE_QUANT_GGUF_IQ2_XS, 256, 74}, {18, TE_QUANT_GGUF_IQ3_XXS, 256, 98},
    {20, TE_QUANT_GGUF_IQ4_NL, 256, 50}, {21, TE_QUANT_GGUF_IQ3_S, 256, 110},
    {23, TE_QUANT_GGUF_IQ4_XS, 256, 136}, {30, TE_QUANT_BF16, 1, 2},
};

const TypeInfo *type_info(uint32_t t) {
    for (const TypeInfo &i : kTypes) {
        if (i.ggml == t) {
            return &i;
        }
    }
    return nullptr;
}

struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t dims[4] = {0, 0, 0, 0};
    uint32_t ggml_type = 0;
    te_quant_kind quant = TE_QUANT_UNKNOWN;
    uint64_t elements = 1, bytes = 0, rel = 0, abs = 0;
    bool sized = false;  // a known type: `bytes` is set
};

struct Kv {
    std::string key;
    uint32_t type;
    uint64_t pos;  // of the value
};

struct Token {
    std::string text;
    int32_t type = 0;
    bool special = false;
};

// Bounds-checked little-endian reads over the mapping.
struct Cursor {
    const uint8_t *p;
    uint64_t size, pos;
    bool skip(uint64_t n) {
        if (pos > size || n > size - pos) {
            return false;
        }
        pos += n;
        return true;
    }
    bool read(void *out, uint64_t n) {
        if (pos > size || n > size - pos) {
            return false;
        }
        memcpy(out, p + pos, n);
        pos += n;
        return true;
    }
    bool u32(uint32_t &v) { return read(&v, 4); }
    bool u64(uint64_t &v) { return read(&v, 8); }
    bool str(std::string &s, uint64_t max_len) {
        uint64_t n;
        if (!u64(n) || n > max_len || pos > size || n > size - pos) {
            return false;
        }
        s.assign(reinterpret_cast<const char *>(p) + pos, n);
        pos += n;
        return true;
    }
};

uint64_t fixed_size(uint32_t type) {
    switch (type) {
        case kU8: case kI8: case kBool: return 1;
        case kU16: case kI16: return 2;
        case kU32: case kI32: case kF32: return 4;
        case kU64: case kI64: case kF64: return 8;
        default: return 0;
    }
}

// Past one value; arrays may nest up to 8 deep (gguf.c:719-755).
te_status skip_value(Cursor &c, uint32_t type, uint32_t depth) {
    if (depth > 8) {
        return TE_STATUS_UNSUPPORTED;
    }
    if (const uint64_t n = fixed_size(type)) {
        return c.skip(n) ? TE_STATUS_OK : TE_STATUS_RUNTIME_ERROR;
    }
    if (type == kStr) {
        uint64_t n;
        return c.u64(n) && c.skip(n) ? TE_STATUS_OK : TE_STATUS_RUNTIME_ERROR;
    }
    if (type != kArr) {
        return TE_STATUS_UNSUPPORTED;
    }
    uint32_t et;
    uint64_t n;
    if (!c.u32(et) || !c.u64(n)) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    if (const uint64_t es = fixed_size(et)) {
        if (n != 0 && es > UINT64_MAX / n) {
            return TE_STATUS_RUNTIME_ERROR;
        }
        return c.skip(n * es) ? TE_STATUS_OK : TE_STATUS_RUNTIME_ERROR;
    }
    for (uint64_t i = 0; i < n; ++i) {
        const te_status s = skip_value(c, et, depth + 1);
        if (s != TE_STATUS_OK) {
            return s;
        }
    }
    return TE_STATUS_OK;
}

// Strings are handled as C strings, as the reference stores them: a string
// with a NUL byte ends there.
void as_c_string(std::string &s) {
    s.resize(strlen(s.c_str()));
}

}  // namespace

struct te_model {
    std::string path;
    te_runtime_options options;
    void *mapping = nullptr;
    size_t mapping_len = 0;
    te_model_info info;
    te_tokenizer_info tok;
    uint64_t alignment = 32;
    std::vector<Kv> kvs;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> tensor_index;
    std::vector<Token> tokens;
    std::vector<std::string> merges;
    std::unordered_map<std::string, uint32_t> token_to_id, merge_rank;
    std::vector<uint32_t> special_ids;  // special tokens, longest text first
    // the file in HBM, made on the first GPU use
    std::mutex gpu_mutex;
    unsigned char *d_mapping = nullptr;
};

namespace {

const Kv *find_kv(const te_model *m, const std::string &key) {
    for (const Kv &kv : m->kvs) {
        if (kv.key == key) {
            return &kv;
        }
    }
    return nullptr;
}

Cursor value_cursor(const te_model *m, const Kv *kv) {
    return Cursor{static_cast<const uint8_t *>(m->mapping), m->mapping_len, kv->pos};
}

// A non-negative integer of type u32, u64, i32 or i64 (gguf.c:821-854).
bool get_u64(const te_model *m, const Kv *kv, uint64_t &out) {
    if (kv == nullptr) {
        return false;
    }
    Cursor c = value_cursor(m, kv);
    switch (kv->type) {
        case kU32: { uint32_t v; if (!c.u32(v)) return false; out = v; return true; }
        case kU64: return c.u64(out);
        case kI32: { int32_t v; if (!c.read(&v, 4) || v < 0) return false; out = (uint64_t)v; return true; }
        case kI64: { int64_t v; if (!c.read(&v, 8) || v < 0) return false; out = (uint64_t)v; return true; }
        default: return false;
    }
}

bool get_f32(const te_model *m, const Kv *kv, float &out) {
    if (kv == nullptr) {
        return false;
    }
    Cursor c = value_cursor(m, kv);
    if (kv->type == kF32) {
        return c.read(&out, 4);
    }
    if (kv->type == kF64) {
        double d;
        if (!c.read(&d, 8)) {
            return false;
        }
        out = (float)d;
        return true;
    }
    return false;
}

bool get_string(const te_model *m, const Kv *kv, std::string &out) {
    if (kv == nullptr || kv->type != kStr) {
        return false;
    }
    Cursor c = value_cursor(m, kv);
    return c.str(out, kMaxString);
}

// Element type and count of an array value; the cursor is left on element 0.
bool get_array(const te_model *m, const Kv *kv, uint32_t &et, uint64_t &n, Cursor &c) {
    if (kv == nullptr || kv->type != kArr) {
        return false;
    }
    c = value_cursor(m, kv);
    return c.u32(et) && c.u64(n);
}

void copy_str(char *dst, size_t cap, const std::string &s) {
    const size_t n = std::min(cap - 1, s.size());
    memcpy(dst, s.data(), n);
    dst[n] = '\0';
}

// "<arch>.<key>" lookups; keys of 128 bytes or more are not looked up
// (gguf.c:1002-1037).
const Kv *prefixed(const te_model *m, const std::string &prefix, const char *key) {
    const std::string k = prefix + key;
    return k.size() < 128 ? find_kv(m, k) : nullptr;
}

bool get_prefixed_u32(const te_model *m, const std::string &prefix, const char *key, uint32_t &out) {
    uint64_t v;
    if (!get_u64(m, prefixed(m, prefix, key), v) || v > 0xffffffffu) {
        return false;
    }
    out = (uint32_t)v;
    return true;
}

// The tokenizer arrays (gguf.c:524-625): tokens and merges must be string
// arrays and token types an int32 array as long as the tokens.
te_status parse_tokenizer_arrays(te_model *m) {
    uint32_t et;
    uint64_t n;
    Cursor c{};
    const Kv *tokens = find_kv(m, "tokenizer.ggml.tokens");
    if (!get_array(m, tokens, et, n, c) || et != kStr) {
        return TE_STATUS_UNSUPPORTED;
    }
    if (n > 0xffffffffu) {
        return TE_STATUS_UNSUPPORTED;
    }
    std::vector<Token> toks(n);
    for (Token &t : toks) {
        if (!c.str(t.text, kMaxString)) {
            return TE_STATUS_RUNTIME_ERROR;
        }
        as_c_string(t.text);
    }
    if (const Kv *types = find_kv(m, "tokenizer.ggml.token_type")) {
        uint64_t tn;
        if (!get_array(m, types, et, tn, c) || et != kI32) {
            return TE_STATUS_UNSUPPORTED;
        }
        std::vector<int32_t> tv(tn);
        for (int32_t &t : tv) {
            if (!c.read(&t, 4)) {
                return TE_STATUS_RUNTIME_ERROR;
            }
        }
        if (tn != n) {
            return TE_STATUS_UNSUPPORTED;
        }
        for (uint64_t i = 0; i < n; ++i) {
            toks[i].type = tv[i];
        }
    }
    std::vector<std::string> merges;
    if (const Kv *mk = find_kv(m, "tokenizer.ggml.merges")) {
        uint64_t mn;
        if (!get_array(m, mk, et, mn, c) || et != kStr) {
            return TE_STATUS_UNSUPPORTED;
        }
        merges.resize(mn);
        for (std::string &s : merges) {
            if (!c.str(s, kMaxString)) {
                return TE_STATUS_RUNTIME_ERROR;
            }
            as_c_string(s);
        }
        if (mn > 0xffffffffu) {
            return TE_STATUS_UNSUPPORTED;
        }
    }
    // control / unknown / user-defined tokens, and <|...|>, are special
    for (Token &t : toks) {
        t.special = t.type != 1 || t.text.compare(0, 2, "<|") == 0;
    }
    m->tokens = std::move(toks);
    m->merges = std::move(merges);
    m->tok.token_count = m->tokens.size();
    m->tok.merge_count = m->merges.size();
    // maps: a repeated key keeps its last value, as the reference's map insert
    m->token_to_id.reserve(m->tokens.size());
    for (size_t i = 0; i < m->tokens.size(); ++i) {
        m->token_to_id[m->tokens[i].text] = (uint32_t)i;
        if (m->tokens[i].special && !m->tokens[i].text.empty()) {
            m->special_ids.push_back((uint32_t)i);
        }
    }
    // longest first; the lower id first among equal lengths
    std::stable_sort(m->special_ids.begin(), m->special_ids.end(), [m](uint32_t a, uint32_t b) {
        return m->tokens[a].text.size() > m->tokens[b].text.size();
    });
    m->merge_rank.reserve(m->merges.size());
    for (size_t i = 0; i < m->merges.size(); ++i) {
        m->merge_rank[m->merges[i]] = (uint32_t)i;
    }
    return TE_STATUS_OK;
}

// Model and tokenizer info from the metadata (gguf.c:371-522).  It runs
// before the tensor table is read (`with_tensors` false: no shape checks)
// and again after it.
te_status extract_info(te_model *m, bool with_tensors) {
    te_model_info &info = m->info;
    te_tokenizer_info &tok = m->tok;
    tok.abi_version = TE_ABI_VERSION;
    std::string s;
    if (get_string(m, find_kv(m, "general.name"), s)) {
        copy_str(info.name, sizeof(info.name), s);
    }
    if (!get_string(m, find_kv(m, "general.architecture"), s)) {
        return TE_STATUS_UNSUPPORTED;
    }
    copy_str(info.architecture, sizeof(info.architecture), s);
    uint64_t alignment = 32;
    if (get_u64(m, find_kv(m, "general.alignment"), alignment) &&
        (alignment == 0 || alignment > (1u << 20) || (alignment & (alignment - 1)) != 0)) {
        return TE_STATUS_UNSUPPORTED;
    }
    m->alignment = alignment;
    const std::string prefix = std::string(info.architecture) + ".";
    if (prefix.size() >= 64) {
        return TE_STATUS_UNSUPPORTED;
    }
    get_prefixed_u32(m, prefix, "context_length", info.context_length);
    get_prefixed_u32(m, prefix, "embedding_length", info.embedding_length);
    get_prefixed_u32(m, prefix, "block_count", info.block_count);
    get_prefixed_u32(m, prefix, "feed_forward_length", info.feed_forward_length);
    get_prefixed_u32(m, prefix, "attention.head_count", info.attention_head_count);
    if (!get_prefixed_u32(m, prefix, "attention.head_count_kv", info.attention_head_count_kv)) {
        info.attention_head_count_kv = info.attention_head_count;
    }
    get_f32(m, prefixed(m, prefix, "attention.layer_norm_rms_epsilon"), info.rms_norm_epsilon);
    if (!get_f32(m, prefixed(m, prefix, "rope.freq_base"), info.rope_freq_base)) {
        info.rope_freq_base = strcmp(info.architecture, "qwen2") == 0 ? 1000000.0f : 10000.0f;
    }
    if (info.embedding_length != 0 && info.attention_head_count != 0) {
        if (with_tensors && info.embedding_length % info.attention_head_count != 0) {
            return TE_STATUS_UNSUPPORTED;
        }
        info.head_dim = info.embedding_length / info.attention_head_count;
    }

    uint32_t et;
    uint64_t n = 0, count;
    Cursor c{};
    if (get_array(m, find_kv(m, "tokenizer.ggml.tokens"), et, n, c) && et == kStr && n <= 0xffffffffu) {
        info.vocab_size = (uint32_t)n;
    }
    tok.token_count = n;
    if (m->tokens.empty() && n != 0) {
        const te_status st = parse_tokenizer_arrays(m);
        if (st != TE_STATUS_OK) {
            return st;
        }
    }
    if (get_array(m, find_kv(m, "tokenizer.ggml.token_type"), et, count, c) && (et == kI32 || et == kU32)) {
        tok.token_type_count = count;
    }
    if (get_array(m, find_kv(m, "tokenizer.ggml.merges"), et, count, c) && et == kStr) {
        tok.merge_count = count;
    }
    if (get_string(m, find_kv(m, "tokenizer.ggml.model"), s)) {
        copy_str(tok.model, sizeof(tok.model), s);
    }
    if (get_string(m, find_kv(m, "tokenizer.ggml.pre"), s)) {
        copy_str(tok.pre, sizeof(tok.pre), s);
    }
    uint64_t id;
    if (get_u64(m, find_kv(m, "tokenizer.ggml.bos_token_id"), id) && id <= 0xffffffffu) {
        tok.bos_token_id = (uint32_t)id;
    }
    if (get_u64(m, find_kv(m, "tokenizer.ggml.eos_token_id"), id) && id <= 0xffffffffu) {
        tok.eos_token_id = (uint32_t)id;
    }
    if (get_u64(m, find_kv(m, "tokenizer.ggml.padding_token_id"), id) && id <= 0xffffffffu) {
        tok.padding_token_id = (uint32_t)id;
    }
    if (const Kv *kv = find_kv(m, "tokenizer.ggml.add_bos_token"); kv != nullptr && kv->type == kBool) {
        Cursor b = value_cursor(m, kv);
        uint8_t v;
        if (b.read(&v, 1)) {
            tok.add_bos_token = v != 0;
        }
    }
    if (!with_tensors) {
        return TE_STATUS_OK;
    }
    auto it = m->tensor_index.find("token_embd.weight");
    if (it != m->tensor_index.end()) {
        const Tensor &e = m->tensors[it->second];
        if (e.n_dims >= 2 && e.dims[1] <= 0xffffffffu) {
            if (info.vocab_size == 0) {
                info.vocab_size = (uint32_t)e.dims[1];
            }
            if (info.embedding_length == 0 && e.dims[0] <= 0xffffffffu) {
                info.embedding_length = (uint32_t)e.dims[0];
            }
        }
    }
    if (info.embedding_length == 0 || info.block_count == 0 || info.feed_forward_length == 0 ||
        info.attention_head_count == 0 || info.attention_head_count_kv == 0 || info.vocab_size == 0 ||
        info.rms_norm_epsilon == 0.0f) {
        return TE_STATUS_UNSUPPORTED;
    }
    return TE_STATUS_OK;
}

// Header, metadata, tensor table (gguf.c:221-369).
te_status parse_gguf(te_model *m) {
    Cursor c{static_cast<const uint8_t *>(m->mapping), m->mapping_len, 0};
    te_model_info &info = m->info;
    uint32_t magic;
    uint64_t n_tensors, n_kv;
    if (!c.u32(magic) || !c.u32(info.gguf_version) || !c.u64(n_tensors) || !c.u64(n_kv)) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    if (magic != 0x46554747u || info.gguf_version < 2 || info.gguf_version > 3) {
        return TE_STATUS_UNSUPPORTED;
    }
    if (n_kv > kMaxCount || n_tensors > kMaxCount) {
        return TE_STATUS_UNSUPPORTED;
    }
    info.abi_version = TE_ABI_VERSION;
    info.metadata_kv_count = n_kv;
    info.tensor_count = n_tensors;
    info.file_size_bytes = m->mapping_len;
    m->kvs.resize(n_kv);
    for (Kv &kv : m->kvs) {
        if (!c.str(kv.key, kMaxName) || !c.u32(kv.type)) {
            return TE_STATUS_RUNTIME_ERROR;
        }
        kv.pos = c.pos;
        const te_status s = skip_value(c, kv.type, 0);
        if (s != TE_STATUS_OK) {
            return s;
        }
    }
    te_status s = extract_info(m, false);
    if (s != TE_STATUS_OK) {
        return s;
    }
    m->tensors.resize(n_tensors);
    for (Tensor &t : m->tensors) {
        if (!c.str(t.name, kMaxName)) {
            return TE_STATUS_RUNTIME_ERROR;
        }
        as_c_string(t.name);
        if (!c.u32(t.n_dims) || t.n_dims == 0 || t.n_dims > 4) {
            return TE_STATUS_UNSUPPORTED;
        }
        for (uint32_t d = 0; d < t.n_dims; ++d) {
            if (!c.u64(t.dims[d]) || t.dims[d] == 0 || t.elements > UINT64_MAX / t.dims[d]) {
                return TE_STATUS_RUNTIME_ERROR;
            }
            t.elements *= t.dims[d];
        }
        if (!c.u32(t.ggml_type) || !c.u64(t.rel)) {
            return TE_STATUS_RUNTIME_ERROR;
        }
        const TypeInfo *ti = type_info(t.ggml_type);
        t.quant = ti != nullptr ? ti->quant : TE_QUANT_UNKNOWN;
        if (t.quant > TE_QUANT_UNKNOWN && t.quant < TE_QUANT_COUNT) {
            info.quant_tensor_counts[t.quant] += 1;
        }
        if (info.parameter_count > UINT64_MAX - t.elements) {
            return TE_STATUS_RUNTIME_ERROR;
        }
        info.parameter_count += t.elements;
        if (ti != nullptr) {
            const uint64_t blocks = (t.elements + ti->block_elems - 1) / ti->block_elems;
            if (blocks > UINT64_MAX / ti->block_bytes) {
                continue;  // no size: the reference leaves such a tensor unsized
            }
            t.bytes = blocks * ti->block_bytes;
            t.sized = true;
            if (info.tensor_data_bytes > UINT64_MAX - t.bytes) {
                return TE_STATUS_RUNTIME_ERROR;
            }
            info.tensor_data_bytes += t.bytes;
        }
    }
    if (c.pos > UINT64_MAX - (m->alignment - 1)) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    info.tensor_data_offset = (c.pos + m->alignment - 1) / m->alignment * m->alignment;
    for (size_t i = 0; i < m->tensors.size(); ++i) {
        Tensor &t = m->tensors[i];
        if (t.rel > UINT64_MAX - info.tensor_data_offset) {
            return TE_STATUS_RUNTIME_ERROR;
        }
        t.abs = info.tensor_data_offset + t.rel;
        if (t.bytes != 0 && (t.abs > m->mapping_len || t.bytes > m->mapping_len - t.abs)) {
            return TE_STATUS_RUNTIME_ERROR;
        }
        m->tensor_index.emplace(t.name, i);  // the first tensor of a name wins, as a linear search
    }
    return extract_info(m, true);
}

const Tensor *find_tensor(const te_model *m, const char *name) {
    auto it = m->tensor_index.find(name);
    return it == m->tensor_index.end() ? nullptr : &m->tensors[it->second];
}

// The tensor's bytes inside the file.
bool tensor_in_file(const te_model *m, const Tensor *t) {
    return t->sized && t->abs <= m->mapping_len && t->bytes <= m->mapping_len - t->abs;
}

te_status require_output(size_t required, const void *out, size_t capacity, size_t *written) {
    if (written == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    *written = required;
    return out == nullptr || capacity < required ? TE_STATUS_INVALID_ARGUMENT : TE_STATUS_OK;
}

te_status rank2(const Tensor *t, size_t &cols, size_t &rows) {
    if (t->n_dims != 2) {
        return TE_STATUS_UNSUPPORTED;
    }
    cols = (size_t)t->dims[0];
    rows = (size_t)t->dims[1];
    return TE_STATUS_OK;
}

// The model file in HBM (copied once; the caller holds no lock).
te_status ensure_device(te_model *m) {
    std::lock_guard<std::mutex> lock(m->gpu_mutex);
    if (m->d_mapping != nullptr) {
        return TE_STATUS_OK;
    }
    if (!te_hip_available()) {
        return TE_STATUS_UNSUPPORTED;
    }
    unsigned char *d = nullptr;
    if (hipMalloc(&d, m->mapping_len) != hipSuccess) {
        return TE_STATUS_OUT_OF_MEMORY;
    }
    if (hipMemcpy(d, m->mapping, m->mapping_len, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d);
        return TE_STATUS_RUNTIME_ERROR;
    }
    m->d_mapping = d;
    return TE_STATUS_OK;
}

// ---- byte-level BPE (reference tokenizer.c) ---------------------------------

// The GPT-2 byte alphabet: printable bytes stand for themselves, the other 68
// map to 256, 257, ... in byte order.
bool gpt2_identity(uint32_t b) { return (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255); }

struct ByteAlphabet {
    uint32_t to_cp[256];
    std::unordered_map<uint32_t, uint8_t> from_cp;
    ByteAlphabet() {
        uint32_t extra = 0;
        for (uint32_t b = 0; b < 256; ++b) {
            to_cp[b] = gpt2_identity(b) ? b : 256 + extra++;
            from_cp[to_cp[b]] = (uint8_t)b;
        }
    }
};

const ByteAlphabet &alphabet() {
    static const ByteAlphabet a;
    return a;
}

void utf8_append(std::string &s, uint32_t cp) {
    if (cp < 0x80) {
        s += (char)cp;
    } else if (cp < 0x800) {
        s += (char)(0xc0 | (cp >> 6));
        s += (char)(0x80 | (cp & 0x3f));
    } else if (cp < 0x10000) {
        s += (char)(0xe0 | (cp >> 12));
        s += (char)(0x80 | ((cp >> 6) & 0x3f));
        s += (char)(0x80 | (cp & 0x3f));
    } else {
        s += (char)(0xf0 | (cp >> 18));
        s += (char)(0x80 | ((cp >> 12) & 0x3f));
        s += (char)(0x80 | ((cp >> 6) & 0x3f));
        s += (char)(0x80 | (cp & 0x3f));
    }
}

// One code point at s[pos]: the lead byte gives the length (1-4) and the
// continuation bytes must be 10xxxxxx; overlong forms are accepted, as the
// reference's decoder does (tokenizer.c:575-612).
bool utf8_next(const std::string &s, size_t &pos, uint32_t &cp) {
    const unsigned char c0 = (unsigned char)s[pos];
    size_t need;
    if (c0 < 0x80) {
        cp = c0;
        pos += 1;
        return true;
    } else if ((c0 & 0xe0) == 0xc0) {
        need = 2, cp = c0 & 0x1f;
    } else if ((c0 & 0xf0) == 0xe0) {
        need = 3, cp = c0 & 0x0f;
    } else if ((c0 & 0xf8) == 0xf0) {
        need = 4, cp = c0 & 0x07;
    } else {
        return false;
    }
    if (need > s.size() - pos) {
        return false;
    }
    for (size_t i = 1; i < need; ++i) {
        const unsigned char ci = (unsigned char)s[pos + i];
        if ((ci & 0xc0) != 0x80) {
            return false;
        }
        cp = cp << 6 | (ci & 0x3f);
    }
    pos += need;
    return true;
}

// The longest special token starting at text[pos] (only at '<').
bool special_at(const te_model *m, const char *text, size_t pos, uint32_t &id, size_t &len) {
    if (text[pos] != '<') {
        return false;
    }
    for (uint32_t sid : m->special_ids) {
        const std::string &t = m->tokens[sid].text;
        if (!t.empty() && strncmp(text + pos, t.c_str(), t.size()) == 0) {
            id = sid;
            len = t.size();
            return true;
        }
    }
    return false;
}

// BPE of one segment: its bytes as GPT-2 symbols, then the adjacent pair of
// lowest merge rank (the leftmost on a tie) merged until none has a rank.
te_status bpe_segment(const te_model *m, const unsigned char *bytes, size_t len, std::vector<uint32_t> &out) {
    std::vector<std::string> sym(len);
    for (size_t i = 0; i < len; ++i) {
        utf8_append(sym[i], alphabet().to_cp[bytes[i]]);
    }
    std::string key;
    while (sym.size() > 1) {
        bool found = false;
        uint32_t best = 0;
        size_t at = 0;
        for (size_t i = 0; i + 1 < sym.size(); ++i) {
            key.assign(sym[i]);
            key += ' ';
            key += sym[i + 1];
            auto it = m->merge_rank.find(key);
            if (it != m->merge_rank.end() && (!found || it->second < best)) {
                found = true;
                best = it->second;
                at = i;
            }
        }
        if (!found) {
            break;
        }
        sym[at] += sym[at + 1];
        sym.erase(sym.begin() + at + 1);
    }
    for (const std::string &s : sym) {
        auto it = m->token_to_id.find(s);
        if (it == m->token_to_id.end()) {
            return TE_STATUS_RUNTIME_ERROR;
        }
        out.push_back(it->second);
    }
    return TE_STATUS_OK;
}

te_status tokenize(const te_model *m, const char *text, int parse_special, std::vector<uint32_t> &out) {
    const size_t n = strlen(text);
    size_t pos = 0;
    while (pos < n) {
        uint32_t id;
        size_t len;
        if (parse_special && special_at(m, text, pos, id, len)) {
            out.push_back(id);
            pos += len;
            continue;
        }
        size_t end = n;
        if (parse_special) {
            for (size_t scan = pos + 1; scan < n; ++scan) {
                if (special_at(m, text, scan, id, len)) {
                    end = scan;
                    break;
                }
            }
        }
        const te_status st = bpe_segment(m, reinterpret_cast<const unsigned char *>(text) + pos, end - pos, out);
        if (st != TE_STATUS_OK) {
            return st;
        }
        pos = end;
    }
    return TE_STATUS_OK;
}

// Token texts back to bytes: GPT-2 alphabet code points become their byte,
// others stay UTF-8.
te_status detokenize(const te_model *m, const uint32_t *ids, size_t count, int skip_special, std::string &out) {
    for (size_t k = 0; k < count; ++k) {
        if (ids[k] >= m->tokens.size()) {
            return TE_STATUS_INVALID_ARGUMENT;
        }
        const Token &t = m->tokens[ids[k]];
        if (skip_special && t.special) {
            continue;
        }
        size_t pos = 0;
        while (pos < t.text.size()) {
            uint32_t cp;
            if (!utf8_next(t.text, pos, cp)) {
                return TE_STATUS_RUNTIME_ERROR;
            }
            auto it = alphabet().from_cp.find(cp);
            if (it != alphabet().from_cp.end()) {
                out += (char)it->second;
            } else if (cp <= 0x10ffff) {
                utf8_append(out, cp);
            } else {
                return TE_STATUS_RUNTIME_ERROR;  // not encodable again
            }
        }
    }
    return TE_STATUS_OK;
}

}  // namespace

// ---- model entry points ------------------------------------------------------

extern "C" te_status te_model_load_gguf(const char *path, const te_runtime_options *options, te_model **out_model) {
    if (path == nullptr || out_model == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    *out_model = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        return TE_STATUS_IO_ERROR;
    }
    // the options must make a kernel plan (tinyengine.c:290-295)
    const te_runtime_options opts = options != nullptr ? *options : te_default_options();
    te_kernel_plan plan;
    const te_status ps = te_make_kernel_plan(&opts, &plan);
    if (ps != TE_STATUS_OK) {
        close(fd);
        return ps;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        return TE_STATUS_IO_ERROR;
    }
    void *map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) {
        return TE_STATUS_IO_ERROR;
    }
    te_model *m = new (std::nothrow) te_model();
    if (m == nullptr) {
        munmap(map, (size_t)st.st_size);
        return TE_STATUS_OUT_OF_MEMORY;
    }
    memset(&m->info, 0, sizeof(m->info));
    memset(&m->tok, 0, sizeof(m->tok));
    m->path = path;
    m->options = opts;
    m->mapping = map;
    m->mapping_len = (size_t)st.st_size;
    te_status s;
    try {
        s = parse_gguf(m);
    } catch (const std::bad_alloc &) {
        s = TE_STATUS_OUT_OF_MEMORY;
    }
    if (s != TE_STATUS_OK) {
        te_model_free(m);
        return s;
    }
    *out_model = m;
    return TE_STATUS_OK;
}

extern "C" te_status te_model_get_info(const te_model *model, te_model_info *out_info) {
    if (model == nullptr || out_info == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    *out_info = model->info;
    return TE_STATUS_OK;
}

extern "C" te_status te_model_get_tokenizer_info(const te_model *model, te_tokenizer_info *out_info) {
    if (model == nullptr || out_info == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    *out_info = model->tok;
    return TE_STATUS_OK;
}

extern "C" te_status te_model_get_tensor_info(const te_model *model, const char *name, te_tensor_info *out_info) {
    if (model == nullptr || name == nullptr || out_info == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    const Tensor *t = find_tensor(model, name);
    if (t == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    memset(out_info, 0, sizeof(*out_info));
    out_info->abi_version = TE_ABI_VERSION;
    out_info->quant = t->quant;
    out_info->ggml_type = t->ggml_type;
    out_info->n_dims = t->n_dims;
    for (uint32_t d = 0; d < t->n_dims && d < 4; ++d) {
        out_info->dims[d] = t->dims[d];
    }
    out_info->elements = t->elements;
    out_info->bytes = t->bytes;
    out_info->relative_offset = t->rel;
    out_info->absolute_offset = t->abs;
    copy_str(out_info->name, sizeof(out_info->name), t->name);
    return TE_STATUS_OK;
}

extern "C" te_status te_format_qwen_chat_prompt(const char *prompt, char *out, size_t out_capacity,
                                                size_t *out_written) {
    static const char prefix[] = "<|im_start|>user\n";
    static const char suffix[] = "<|im_end|>\n<|im_start|>assistant\n";
    if (prompt == nullptr || out_written == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    const size_t n = strlen(prompt);
    const size_t required = sizeof(prefix) - 1 + n + sizeof(suffix) - 1;
    *out_written = required;
    if (out == nullptr || out_capacity <= required) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    memcpy(out, prefix, sizeof(prefix) - 1);
    memcpy(out + sizeof(prefix) - 1, prompt, n);
    memcpy(out + sizeof(prefix) - 1 + n, suffix, sizeof(suffix));  // with the terminator
    return TE_STATUS_OK;
}

extern "C" te_status te_model_tokenize(const te_model *model, const char *text, int parse_special,
                                       uint32_t *out_tokens, size_t out_capacity, size_t *out_written) {
    if (model == nullptr || text == nullptr || out_written == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (model->tokens.empty()) {
        return TE_STATUS_UNSUPPORTED;
    }
    std::vector<uint32_t> ids;
    te_status s;
    try {
        s = tokenize(model, text, parse_special, ids);
    } catch (const std::bad_alloc &) {
        return TE_STATUS_OUT_OF_MEMORY;
    }
    if (s != TE_STATUS_OK) {
        return s;
    }
    *out_written = ids.size();
    if (out_tokens == nullptr || out_capacity < ids.size()) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    std::copy(ids.begin(), ids.end(), out_tokens);
    return TE_STATUS_OK;
}

extern "C" te_status te_model_detokenize(const te_model *model, const uint32_t *tokens, size_t token_count,
                                         int skip_special, char *out, size_t out_capacity, size_t *out_written) {
    if (model == nullptr || tokens == nullptr || out_written == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (model->tokens.empty()) {
        return TE_STATUS_UNSUPPORTED;
    }
    if (out != nullptr && out_capacity != 0) {
        out[0] = '\0';
    }
    std::string text;
    te_status s;
    try {
        s = detokenize(model, tokens, token_count, skip_special, text);
    } catch (const std::bad_alloc &) {
        return TE_STATUS_OUT_OF_MEMORY;
    }
    if (s != TE_STATUS_OK) {
        return s;
    }
    *out_written = text.size();
    if (out == nullptr || out_capacity <= text.size()) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    memcpy(out, text.c_str(), text.size() + 1);
    return TE_STATUS_OK;
}

extern "C" te_status te_model_read_f32_tensor(const te_model *model, const char *name, float *out,
                                              size_t out_capacity, size_t *out_written) {
    if (model == nullptr || name == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    const Tensor *t = find_tensor(model, name);
    if (t == nullptr || t->ggml_type != 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    const te_status s = require_output((size_t)t->elements, out, out_capacity, out_written);
    if (s != TE_STATUS_OK) {
        return s;
    }
    if (!tensor_in_file(model, t)) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    memcpy(out, static_cast<const unsigned char *>(model->mapping) + t->abs, t->elements * sizeof(float));
    return TE_STATUS_OK;
}

extern "C" te_status te_model_dequantize_row_f32(const te_model *model, const char *name, uint64_t row_index,
                                                 float *out, size_t out_capacity, size_t *out_written) {
    if (model == nullptr || name == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    const Tensor *t = find_tensor(model, name);
    if (t == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    size_t cols, rows;
    te_status s = rank2(t, cols, rows);
    if (s != TE_STATUS_OK) {
        return s;
    }
    if (row_index >= rows) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    s = require_output(cols, out, out_capacity, out_written);
    if (s != TE_STATUS_OK) {
        return s;
    }
    if (!tensor_in_file(model, t)) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    if (t->ggml_type != 0 && te_hip::ggml_row_bytes(t->ggml_type, cols) == 0) {
        return TE_STATUS_UNSUPPORTED;  // other types; Q4_0 / Q8_0 rows not whole blocks
    }
    te_model *m = const_cast<te_model *>(model);  // the device copy is a cache
    if ((s = ensure_device(m)) != TE_STATUS_OK) {
        return s;
    }
    float *d = nullptr;
    if (hipMalloc(&d, cols * sizeof(float)) != hipSuccess) {
        return TE_STATUS_OUT_OF_MEMORY;
    }
    s = te_hip::launch_dequant_row(m->d_mapping + t->abs, t->ggml_type, cols, row_index, d, nullptr);
    if (s == TE_STATUS_OK && hipMemcpy(out, d, cols * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) {
        s = TE_STATUS_RUNTIME_ERROR;
    }
    (void)hipFree(d);
    return s;
}

extern "C" te_status te_model_matvec_f32(const te_model *model, const char *name, const float *input,
                                         size_t input_len, float *out, size_t out_capacity, size_t *out_written) {
    if (model == nullptr || name == nullptr || input == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    const Tensor *t = find_tensor(model, name);
    if (t == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    size_t cols, rows;
    te_status s = rank2(t, cols, rows);
    if (s != TE_STATUS_OK) {
        return s;
    }
    if (input_len != cols) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    s = require_output(rows, out, out_capacity, out_written);
    if (s != TE_STATUS_OK) {
        return s;
    }
    if (!tensor_in_file(model, t)) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    const uint32_t type = t->ggml_type;
    if (type != 0 && te_hip::ggml_row_bytes(type, cols) == 0) {
        return TE_STATUS_UNSUPPORTED;  // other types; Q4_0 / Q8_0 rows not whole blocks
    }
    if (rows > (1u << 30) || cols > (1u << 24)) {
        return TE_STATUS_UNSUPPORTED;
    }
    te_model *m = const_cast<te_model *>(model);
    if ((s = ensure_device(m)) != TE_STATUS_OK) {
        return s;
    }
    // The GEMV kernels read Q4_0 / Q8_0 rows from 4-byte and F32 rows from
    // 16-byte aligned addresses, F32 rows in float4 steps.  A tensor that does
    // not start so (GGUF alignment below 4 / 16), or F32 rows of a width not a
    // multiple of 4, run from an aligned copy, F32 rows zero-padded to a
    // multiple of 4 together with the input: the padding adds 0 * 0 to each row.
    const size_t pcols = type == 0 ? (cols + 3) / 4 * 4 : cols;
    const bool stage = type == 0 ? (t->abs % 16 != 0 || pcols != cols) : t->abs % 4 != 0;
    const size_t wbytes = type == 0 ? rows * pcols * sizeof(float) : (size_t)t->bytes;
    const size_t in_off = stage ? (wbytes + 255) / 256 * 256 : 0;
    const size_t bytes = in_off + (pcols + rows) * sizeof(float);
    unsigned char *buf = nullptr;
    if (hipMalloc(&buf, bytes) != hipSuccess) {
        return TE_STATUS_OUT_OF_MEMORY;
    }
    float *x = reinterpret_cast<float *>(buf + in_off);
    const unsigned char *w = m->d_mapping + t->abs;
    bool ok = true;
    if (stage) {
        if (type == 0) {
            ok = hipMemset(buf, 0, wbytes) == hipSuccess &&
                 hipMemcpy2D(buf, pcols * sizeof(float), w, cols * sizeof(float), cols * sizeof(float), rows,
                             hipMemcpyDeviceToDevice) == hipSuccess;
        } else {
            ok = hipMemcpy(buf, w, wbytes, hipMemcpyDeviceToDevice) == hipSuccess;
        }
        w = buf;
    }
    ok = ok && hipMemset(x, 0, pcols * sizeof(float)) == hipSuccess &&
         hipMemcpy(x, input, cols * sizeof(float), hipMemcpyHostToDevice) == hipSuccess;
    s = ok ? te_hip::launch_matvec(w, type, x, pcols, rows, x + pcols, nullptr) : TE_STATUS_RUNTIME_ERROR;
    if (s == TE_STATUS_OK && hipMemcpy(out, x + pcols, rows * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) {
        s = TE_STATUS_RUNTIME_ERROR;
    }
    (void)hipFree(buf);
    return s;
}

extern "C" void te_model_free(te_model *model) {
    if (model == nullptr) {
        return;
    }
    if (model->d_mapping != nullptr) {
        (void)hipFree(model->d_mapping);
    }
    if (model->mapping != nullptr) {
        munmap(model->mapping, model->mapping_len);
    }
    delete model;
}

// ---- context and generation --------------------------------------------------

struct te_context {
    te_model *model = nullptr;
    te_runtime_options options;
    std::mutex mutex;
    // device state for one context length, made on the first generate
    bool ready = false;
    size_t ctx = 0, layers = 0, hidden = 0, kv = 0, heads = 0, kv_heads = 0, head_dim = 0, ffn = 0, vocab = 0;
    uint32_t type = 0, head_type = 0, embd_type = 0;
    uint64_t head_off = 0, embd_off = 0;
    std::vector<uint64_t> offs[7];
    uint16_t *kc = nullptr, *vc = nullptr;
    float *cos = nullptr, *sin = nullptr, *attn_norm = nullptr, *ffn_norm = nullptr, *qb = nullptr, *kb = nullptr,
          *vb = nullptr, *out_norm = nullptr, *hidden_buf = nullptr, *logits = nullptr;
    uint32_t *token = nullptr;
    void *ws = nullptr;
    size_t ws_bytes = 0;
    std::vector<void *> allocations;
    // the tokens whose K / V fill cache positions 0 .. history.size() - 1
    std::vector<uint32_t> history;
    // batched prompt prefill: chunk rows of hidden states, token ids, the
    // layer flow's workspace, and the transposed value copy V^T the prefill
    // attention reads, current for positions 0 .. vt_valid - 1 (the decode
    // path appends to the value cache only; a prefill chunk first brings V^T
    // up to its base position)
    bool batch_ok = false;
    size_t chunk = 0;
    float *px = nullptr;
    uint32_t *pids = nullptr;
    void *pws = nullptr;
    size_t pws_bytes = 0;
    uint16_t *vt = nullptr;
    size_t vt_valid = 0;
    // op-by-op decode (TINYENGINE_FUSED_DECODE_LAYER=0): activations and the
    // split-K workspace, made on first use
    float *ufw = nullptr;
    void *udws = nullptr;
    size_t udws_bytes = 0;
    // sampled decoding's candidate workspace, made on first use
    void *sws = nullptr;
    size_t sws_bytes = 0;
};

namespace {

void release_state(te_context *c) {
    for (void *p : c->allocations) {
        (void)hipFree(p);
    }
    c->allocations.clear();
    c->history.clear();
    c->vt_valid = 0;
    c->ufw = nullptr;
    c->udws = nullptr;
    c->sws = nullptr;
    c->ready = false;
}

// The reference's path switches: NAME=0 turns a fused path off (qwen.c:1392,
// :1484-1491, :1646, :1799).
bool env_off(const char *name) {
    const char *e = getenv(name);
    return e != nullptr && strcmp(e, "0") == 0;
}

template <typename T>
te_status dev_alloc(te_context *c, T **p, size_t count) {
    void *v = nullptr;
    if (hipMalloc(&v, std::max<size_t>(count, 1) * sizeof(T)) != hipSuccess) {
        return TE_STATUS_OUT_OF_MEMORY;
    }
    c->allocations.push_back(v);
    *p = static_cast<T *>(v);
    return TE_STATUS_OK;
}

// A [len] F32 tensor of the model copied (on the device) to dst, with the
// reference's statuses (te_qwen_read_f32_exact, qwen.c:2124-2131): missing or
// not F32 -> INVALID_ARGUMENT, more elements than len -> INVALID_ARGUMENT,
// fewer -> RUNTIME_ERROR.
te_status gather_f32(te_context *c, const char *name, size_t len, float *dst) {
    const Tensor *t = find_tensor(c->model, name);
    if (t == nullptr || t->ggml_type != 0 || t->elements > len) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (t->elements != len || !tensor_in_file(c->model, t)) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    return hipMemcpy(dst, c->model->d_mapping + t->abs, len * sizeof(float), hipMemcpyDeviceToDevice) == hipSuccess
               ? TE_STATUS_OK
               : TE_STATUS_RUNTIME_ERROR;
}

// A [cols][rows] weight matrix of the model: its offset and type.
te_status weight(te_context *c, const char *name, size_t cols, size_t rows, uint64_t &off, uint32_t &type) {
    const Tensor *t = find_tensor(c->model, name);
    if (t == nullptr || t->n_dims != 2 || t->dims[0] != cols || t->dims[1] != rows || !tensor_in_file(c->model, t)) {
        return TE_STATUS_UNSUPPORTED;
    }
    off = t->abs;
    type = t->ggml_type;
    return TE_STATUS_OK;
}

// The model's shapes and the context length, checked as te_qwen_state_init
// does (qwen.c:430-450) for a generation that needs `required` positions.
te_status check_shapes(te_context *c, size_t required) {
    const te_model_info &info = c->model->info;
    if (strcmp(info.architecture, "qwen2") != 0 || info.embedding_length == 0 || info.feed_forward_length == 0 ||
        info.block_count == 0 || info.attention_head_count == 0 || info.attention_head_count_kv == 0 ||
        info.head_dim == 0 || info.vocab_size == 0) {
        return TE_STATUS_UNSUPPORTED;
    }
    const size_t ctx = c->options.context_tokens != 0 ? c->options.context_tokens : 512;
    if (required > ctx || (size_t)info.attention_head_count * info.head_dim != info.embedding_length) {
        return TE_STATUS_UNSUPPORTED;
    }
    return TE_STATUS_OK;
}

// Device state of a Qwen2 model at the context's length (te_qwen_state_init,
// qwen.c:424-577, in HBM): fp16 KV cache [layers][ctx][kv], RoPE tables
// [ctx][head_dim/2], the per-layer norm weights and biases gathered into
// [layers][n] arrays, hidden / logits / token buffers and the decode
// workspace.  Weights stay where they are in the device copy of the file.
te_status init_state(te_context *c) {
    te_model *m = c->model;
    const te_model_info &info = m->info;
    c->hidden = info.embedding_length;
    c->ffn = info.feed_forward_length;
    c->layers = info.block_count;
    c->heads = info.attention_head_count;
    c->kv_heads = info.attention_head_count_kv;
    c->head_dim = info.head_dim;
    c->kv = c->kv_heads * c->head_dim;
    c->vocab = info.vocab_size;
    c->ctx = c->options.context_tokens != 0 ? c->options.context_tokens : 512;
    te_status s = ensure_device(m);
    if (s != TE_STATUS_OK) {
        return s;
    }
    const size_t ln = c->layers * c->hidden, lk = c->layers * c->kv, cache = c->layers * c->ctx * c->kv;
    if ((s = dev_alloc(c, &c->kc, cache)) != TE_STATUS_OK || (s = dev_alloc(c, &c->vc, cache)) != TE_STATUS_OK ||
        (s = dev_alloc(c, &c->cos, c->ctx * c->head_dim / 2)) != TE_STATUS_OK ||
        (s = dev_alloc(c, &c->sin, c->ctx * c->head_dim / 2)) != TE_STATUS_OK ||
        (s = dev_alloc(c, &c->attn_norm, ln)) != TE_STATUS_OK || (s = dev_alloc(c, &c->ffn_norm, ln)) != TE_STATUS_OK ||
        (s = dev_alloc(c, &c->qb, ln)) != TE_STATUS_OK || (s = dev_alloc(c, &c->kb, lk)) != TE_STATUS_OK ||
        (s = dev_alloc(c, &c->vb, lk)) != TE_STATUS_OK || (s = dev_alloc(c, &c->out_norm, c->hidden)) != TE_STATUS_OK ||
        (s = dev_alloc(c, &c->hidden_buf, c->hidden)) != TE_STATUS_OK ||
        (s = dev_alloc(c, &c->logits, c->vocab)) != TE_STATUS_OK || (s = dev_alloc(c, &c->token, 1)) != TE_STATUS_OK) {
        return s;
    }
    char name[96];
    for (size_t l = 0; l < c->layers; ++l) {
        const struct {
            const char *what;
            float *dst;
            size_t len;
        } parts[5] = {{"attn_norm.weight", c->attn_norm + l * c->hidden, c->hidden},
                      {"ffn_norm.weight", c->ffn_norm + l * c->hidden, c->hidden},
                      {"attn_q.bias", c->qb + l * c->hidden, c->hidden},
                      {"attn_k.bias", c->kb + l * c->kv, c->kv},
                      {"attn_v.bias", c->vb + l * c->kv, c->kv}};
        for (const auto &p : parts) {
            snprintf(name, sizeof(name), "blk.%zu.%s", l, p.what);
            if ((s = gather_f32(c, name, p.len, p.dst)) != TE_STATUS_OK) {
                return s;
            }
        }
    }
    if ((s = gather_f32(c, "output_norm.weight", c->hidden, c->out_norm)) != TE_STATUS_OK) {
        return s;
    }
    // the decode slot's weights: one Q4_0 / Q8_0 type for the seven layer matrices
    static const char *const kNames[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                                          "ffn_down"};
    const size_t cols[7] = {c->hidden, c->hidden, c->hidden, c->hidden, c->hidden, c->hidden, c->ffn};
    const size_t rows[7] = {c->hidden, c->kv, c->kv, c->hidden, c->ffn, c->ffn, c->hidden};
    for (int w = 0; w < 7; ++w) {
        c->offs[w].assign(c->layers, 0);
    }
    for (size_t l = 0; l < c->layers; ++l) {
        for (int w = 0; w < 7; ++w) {
            snprintf(name, sizeof(name), "blk.%zu.%s.weight", l, kNames[w]);
            uint32_t t;
            if ((s = weight(c, name, cols[w], rows[w], c->offs[w][l], t)) != TE_STATUS_OK) {
                return s;
            }
            if (l == 0 && w == 0) {
                c->type = t;
            } else if (t != c->type) {
                return TE_STATUS_UNSUPPORTED;
            }
        }
    }
    if ((s = weight(c, "token_embd.weight", c->hidden, c->vocab, c->embd_off, c->embd_type)) != TE_STATUS_OK) {
        return s;
    }
    if (c->embd_type != 0 && te_hip::ggml_row_bytes(c->embd_type, c->hidden) == 0) {
        return TE_STATUS_UNSUPPORTED;
    }
    const char *head = find_tensor(m, "output.weight") != nullptr ? "output.weight" : "token_embd.weight";
    if ((s = weight(c, head, c->hidden, c->vocab, c->head_off, c->head_type)) != TE_STATUS_OK) {
        return s;
    }
    if ((s = te_hip_rope_table_f32(c->cos, c->sin, c->ctx, c->head_dim, info.rope_freq_base)) != TE_STATUS_OK) {
        return s;
    }
    c->ws_bytes = te_hip_decode_all_layers_workspace_bytes(c->ctx - 1, c->hidden, c->kv, c->heads, c->kv_heads,
                                                           c->head_dim, c->ffn, c->vocab);
    unsigned char *ws = nullptr;
    if ((s = dev_alloc(c, &ws, c->ws_bytes)) != TE_STATUS_OK) {
        return s;
    }
    c->ws = ws;
    // batched prefill needs 2-byte aligned layer weights (the GEMM's block reads)
    c->batch_ok = true;
    for (int w = 0; w < 7; ++w) {
        for (size_t l = 0; l < c->layers; ++l) {
            c->batch_ok = c->batch_ok && (c->offs[w][l] & 1u) == 0;
        }
    }
    if (c->batch_ok) {
        c->chunk = std::min<size_t>(512, c->ctx);
        const size_t ch = c->chunk;
        const size_t vt_bytes = te_hip_value_t_bytes(1, c->layers, c->ctx, c->kv_heads, c->head_dim);
        c->pws_bytes = te_hip_prefill_all_layers_workspace_bytes(ch, c->hidden, c->kv, c->ffn);
        unsigned char *pws = nullptr;
        if ((s = dev_alloc(c, &c->px, ch * c->hidden)) != TE_STATUS_OK ||
            (s = dev_alloc(c, &c->pids, ch)) != TE_STATUS_OK ||
            (s = dev_alloc(c, &pws, c->pws_bytes)) != TE_STATUS_OK ||
            (s = dev_alloc(c, &c->vt, vt_bytes / sizeof(uint16_t))) != TE_STATUS_OK) {
            return s;
        }
        c->pws = pws;
        // V^T positions past a sequence must be finite: start from zeros
        if (hipMemset(c->vt, 0, vt_bytes) != hipSuccess) {
            return TE_STATUS_RUNTIME_ERROR;
        }
        c->vt_valid = 0;
    }
    c->ready = true;
    return TE_STATUS_OK;
}

// Prompt tokens ids[start .. end) at positions start .. end - 1, `chunk` rows
// at a time through every layer (te_qwen_prefill_prompt_batch,
// qwen.c:630-905) by te_hip_prefill_all_layers_f16: per layer RMSNorm + Q / K
// / V GEMMs, bias + RoPE + fp16 append + causal MFMA attention from the
// chunk's base position, Wo GEMM + residual, RMSNorm + gate / up GEMMs,
// SwiGLU + down GEMM + residual.  TINYENGINE_PREFILL_ALL_LAYERS=0 runs the
// same flow one layer per call (te_hip_prefill_layer_f16), as the reference's
// switch selects its per-layer Metal path (qwen.c:1646-1649).  The last row's
// hidden state is left in hidden_buf.
te_status prefill_batch(te_context *c, const uint32_t *ids, size_t start, size_t end) {
    te_model *m = c->model;
    const unsigned char *base = m->d_mapping;
    const float eps = m->info.rms_norm_epsilon;
    const size_t H = c->hidden;
    // TINYENGINE_PREFILL_ALL_LAYERS=0: one layer-flow launch sequence per
    // layer; with TINYENGINE_FUSED_PREFILL_LAYER=0 as well no batched path
    // remains and the prompt goes token by token (UNSUPPORTED, as the
    // reference's batch prefill falls back, qwen.c:348-356)
    const bool per_layer = env_off("TINYENGINE_PREFILL_ALL_LAYERS");
    if (per_layer && env_off("TINYENGINE_FUSED_PREFILL_LAYER")) {
        return TE_STATUS_UNSUPPORTED;
    }
    const size_t vt_layer = te_hip_value_t_bytes(1, 1, c->ctx, c->kv_heads, c->head_dim) / sizeof(uint16_t);
    te_status s = TE_STATUS_OK;
    for (size_t p0 = start; p0 < end && s == TE_STATUS_OK; p0 += c->chunk) {
        const size_t M = std::min(c->chunk, end - p0);
        if (hipMemcpy(c->pids, ids + p0, M * sizeof(uint32_t), hipMemcpyHostToDevice) != hipSuccess) {
            return TE_STATUS_RUNTIME_ERROR;
        }
        te_hip::prof_begin(nullptr);
        s = te_hip::launch_dequant_rows(base + c->embd_off, c->embd_type, H, c->pids, M, c->px, nullptr);
        te_hip::prof_mark(nullptr, te_hip::kProfEmbed);
        if (s == TE_STATUS_OK && c->vt_valid < p0) {
            // positions the decode path appended since V^T was last current
            s = te_hip_value_transpose_f16(c->vc, c->vt, 1, c->layers, c->vt_valid, p0 - c->vt_valid, c->ctx,
                                           c->kv_heads, c->head_dim, nullptr);
            te_hip::prof_mark(nullptr, te_hip::kProfAttention);
        }
        if (s != TE_STATUS_OK) {
            break;
        }
        const uint64_t *o[7];
        for (int w = 0; w < 7; ++w) {
            o[w] = c->offs[w].data();
        }
        if (!per_layer) {
            s = te_hip_prefill_all_layers_f16(base, m->mapping_len, o[0], o[1], o[2], o[3], o[4], o[5], o[6],
                                              c->layers, c->type, c->px, c->attn_norm, c->ffn_norm, c->qb, c->kb,
                                              c->vb, c->cos, c->sin, c->kc, c->vc, c->vt, p0, M, c->ctx, H, c->kv,
                                              c->heads, c->kv_heads, c->head_dim, c->ffn, eps, c->px, c->pws,
                                              c->pws_bytes, nullptr);
        } else {
            const size_t ckv = c->ctx * c->kv;
            for (size_t l = 0; l < c->layers && s == TE_STATUS_OK; ++l) {
                s = te_hip_prefill_layer_f16(base, m->mapping_len, o[0][l], o[1][l], o[2][l], o[3][l], o[4][l],
                                             o[5][l], o[6][l], c->type, c->px, c->attn_norm + l * H,
                                             c->ffn_norm + l * H, c->qb + l * H, c->kb + l * c->kv, c->vb + l * c->kv,
                                             c->cos, c->sin, c->kc + l * ckv, c->vc + l * ckv, c->vt + l * vt_layer,
                                             p0, M, c->ctx, H, c->kv, c->heads, c->kv_heads, c->head_dim, c->ffn,
                                             eps, c->px, c->pws, c->pws_bytes, nullptr);
            }
        }
        if (s != TE_STATUS_OK) {
            break;
        }
        c->vt_valid = p0 + M;
        if (p0 + M == end &&
            hipMemcpy(c->hidden_buf, c->px + (M - 1) * H, H * sizeof(float), hipMemcpyDeviceToDevice) !=
                hipSuccess) {
            s = TE_STATUS_RUNTIME_ERROR;
        }
    }
    return s;
}

// Greedy next token from hidden_buf: RMSNorm + lm_head GEMV, then argmax, into c->token.
te_status project_greedy(te_context *c) {
    const te_hip::GemvSeg h = {c->model->d_mapping + c->head_off, c->logits, nullptr, c->vocab};
    float *xtmp = static_cast<float *>(c->ws);
    te_status s = te_hip::launch_gemv(c->head_type, te_hip::kGemvRmsNorm, &h, 1, c->hidden, c->hidden_buf, nullptr,
                                      c->out_norm, c->model->info.rms_norm_epsilon, xtmp,
                                      xtmp + ((std::max(c->hidden, c->ffn) + 63) / 64 * 64), nullptr);
    te_hip::prof_mark(nullptr, te_hip::kProfLmHead);
    if (s == TE_STATUS_OK) {
        s = te_hip::launch_argmax(c->logits, c->vocab, c->token, nullptr);
        te_hip::prof_mark(nullptr, te_hip::kProfElementwise);
    }
    return s;
}

// TINYENGINE_DECODE_ALL_LAYERS=0: one fused decode-layer launch sequence per
// layer (te_hip_decode_layer_f16), then the head.
te_status forward_per_layer(te_context *c, size_t position, bool project) {
    const size_t H = c->hidden, ckv = c->ctx * c->kv;
    te_status s = TE_STATUS_OK;
    for (size_t l = 0; l < c->layers && s == TE_STATUS_OK; ++l) {
        s = te_hip_decode_layer_f16(c->model->d_mapping, c->model->mapping_len, c->offs[0][l], c->offs[1][l],
                                    c->offs[2][l], c->offs[3][l], c->offs[4][l], c->offs[5][l], c->offs[6][l],
                                    c->type, c->hidden_buf, c->attn_norm + l * H, c->ffn_norm + l * H,
                                    c->qb + l * H, c->kb + l * c->kv, c->vb + l * c->kv, c->cos, c->sin,
                                    c->kc + l * ckv, c->vc + l * ckv, position, c->ctx, H, c->kv, c->heads,
                                    c->kv_heads, c->head_dim, c->ffn, c->model->info.rms_norm_epsilon,
                                    c->hidden_buf, c->ws, c->ws_bytes, nullptr);
    }
    return s == TE_STATUS_OK && project ? project_greedy(c) : s;
}

// TINYENGINE_FUSED_DECODE_LAYER=0: the layer as separate operations through
// the public entry points, in the reference's order (qwen.c te_qwen_forward_token):
// RMSNorm, q/k/v GEMVs, the decode step (bias + RoPE + fp16 append + attention),
// Wo GEMV, residual add, RMSNorm, gate/up GEMVs, SwiGLU, down GEMV, residual add.
te_status forward_unfused(te_context *c, size_t position, bool project) {
    const size_t H = c->hidden, KV = c->kv, F = c->ffn, ckv = c->ctx * c->kv;
    te_status s = TE_STATUS_OK;
    if (c->ufw == nullptr) {
        c->udws_bytes = te_hip_attention_decode_workspace_bytes(nullptr, c->ctx - 1, 1, 1, c->heads, c->kv_heads,
                                                                c->head_dim);
        unsigned char *dws = nullptr;
        if (c->udws_bytes == 0 || (s = dev_alloc(c, &c->ufw, 5 * H + 2 * KV + 3 * F)) != TE_STATUS_OK ||
            (s = dev_alloc(c, &dws, c->udws_bytes)) != TE_STATUS_OK) {
            return s != TE_STATUS_OK ? s : TE_STATUS_RUNTIME_ERROR;
        }
        c->udws = dws;
    }
    float *xn = c->ufw, *q = xn + H, *att = q + H, *proj = att + H, *dn = proj + H, *k = dn + H, *v = k + KV;
    float *g = v + KV, *u = g + F, *act = u + F;
    const unsigned char *base = c->model->d_mapping;
    const float eps = c->model->info.rms_norm_epsilon;
    float *x = c->hidden_buf;
    for (size_t l = 0; l < c->layers && s == TE_STATUS_OK; ++l) {
        static const te_hip::ProfPhase kW[7] = {te_hip::kProfQ, te_hip::kProfK, te_hip::kProfV, te_hip::kProfO,
                                                te_hip::kProfGate, te_hip::kProfUp, te_hip::kProfDown};
        auto mv = [&](int w, const float *in, size_t cols, size_t rows, float *out) {
            const te_status r = te_hip_matvec_f32(base + c->offs[w][l], c->type, in, cols, rows, out, nullptr);
            te_hip::prof_mark(nullptr, kW[w]);
            return r;
        };
        auto ew = [](te_status r) {
            te_hip::prof_mark(nullptr, te_hip::kProfElementwise);
            return r;
        };
        if ((s = ew(te_hip_rmsnorm_f32(x, c->attn_norm + l * H, 1, H, eps, xn, nullptr))) != TE_STATUS_OK ||
            (s = mv(0, xn, H, H, q)) != TE_STATUS_OK || (s = mv(1, xn, H, KV, k)) != TE_STATUS_OK ||
            (s = mv(2, xn, H, KV, v)) != TE_STATUS_OK ||
            (s = te_hip_attention_decode_step_f16(q, k, v, c->qb + l * H, c->kb + l * KV, c->vb + l * KV, c->cos,
                                                  c->sin, c->kc + l * ckv, c->vc + l * ckv, nullptr, position, 1, 1,
                                                  c->ctx, c->heads, c->kv_heads, c->head_dim, att, c->udws,
                                                  c->udws_bytes, nullptr)) != TE_STATUS_OK ||
            (te_hip::prof_mark(nullptr, te_hip::kProfAttention), false) ||
            (s = mv(3, att, H, H, proj)) != TE_STATUS_OK ||
            (s = ew(te_hip_add_f32(x, proj, H, x, nullptr))) != TE_STATUS_OK ||
            (s = ew(te_hip_rmsnorm_f32(x, c->ffn_norm + l * H, 1, H, eps, xn, nullptr))) != TE_STATUS_OK ||
            (s = mv(4, xn, H, F, g)) != TE_STATUS_OK || (s = mv(5, xn, H, F, u)) != TE_STATUS_OK ||
            (s = ew(te_hip_swiglu_f32(g, u, F, act, nullptr))) != TE_STATUS_OK ||
            (s = mv(6, act, F, H, dn)) != TE_STATUS_OK) {
            break;
        }
        s = ew(te_hip_add_f32(x, dn, H, x, nullptr));
    }
    return s == TE_STATUS_OK && project ? project_greedy(c) : s;
}

// One token at `position` through every layer; with `project`, also the
// greedy next token into c->token.  TINYENGINE_FUSED_DECODE_LAYER=0 (which
// also turns the all-layers path off, as in the reference) and
// TINYENGINE_DECODE_ALL_LAYERS=0 select the slower paths above.
te_status forward(te_context *c, uint32_t token, size_t position, bool project) {
    te_hip::prof_begin(nullptr);
    const te_status s = te_hip::launch_dequant_row(c->model->d_mapping + c->embd_off, c->embd_type, c->hidden,
                                                   token, c->hidden_buf, nullptr);
    if (s != TE_STATUS_OK) {
        return s;
    }
    te_hip::prof_mark(nullptr, te_hip::kProfEmbed);
    if (env_off("TINYENGINE_FUSED_DECODE_LAYER")) {
        return forward_unfused(c, position, project);
    }
    if (env_off("TINYENGINE_DECODE_ALL_LAYERS")) {
        return forward_per_layer(c, position, project);
    }
    const uint64_t *o[7];
    for (int w = 0; w < 7; ++w) {
        o[w] = c->offs[w].data();
    }
    return te_hip_decode_all_layers_f16(
        c->model->d_mapping, c->model->mapping_len, o[0], o[1], o[2], o[3], o[4], o[5], o[6], c->layers, c->type,
        c->hidden_buf, c->attn_norm, c->ffn_norm, c->qb, c->kb, c->vb, c->cos, c->sin, c->kc, c->vc, position, c->ctx,
        c->hidden, c->kv, c->heads, c->kv_heads, c->head_dim, c->ffn, c->model->info.rms_norm_epsilon, c->hidden_buf,
        c->head_off, c->head_type, project ? c->out_norm : nullptr, project ? c->vocab : 0,
        project ? c->token : nullptr, c->ws, c->ws_bytes, nullptr);
}

struct Sampler {
    float temperature = 0.3f;  // reference defaults (qwen.c:505-507)
    uint32_t top_k = 40;
    uint64_t rng = 0x9e3779b97f4a7c15ULL;
    Sampler() {
        if (const char *e = getenv("TINYENGINE_TEMPERATURE")) {
            const float v = strtof(e, nullptr);
            if (v >= 0.0f && v <= 5.0f) {
                temperature = v;
            }
        }
        if (const char *e = getenv("TINYENGINE_TOP_K")) {
            const long v = strtol(e, nullptr, 10);
            if (v >= 1 && v <= 1000) {
                top_k = (uint32_t)v;
            }
        }
        if (const char *e = getenv("TINYENGINE_SEED")) {
            const unsigned long long v = strtoull(e, nullptr, 10);
            if (v != 0) {
                rng = v;
            }
        }
    }
};

// The next token after the hidden state in c->hidden_buf: greedy from the fused
// head (already in c->token when `greedy_done`), or sampled from the logits.
te_status next_token(te_context *c, Sampler &sm, uint32_t &id) {
    if (sm.temperature > 0.0f) {
        const te_hip::GemvSeg h = {c->model->d_mapping + c->head_off, c->logits, nullptr, c->vocab};
        float *xtmp = static_cast<float *>(c->ws);  // the workspace's first pieces are scratch between tokens
        te_hip::prof_begin(nullptr);
        te_status s = te_hip::launch_gemv(c->head_type, te_hip::kGemvRmsNorm, &h, 1, c->hidden, c->hidden_buf,
                                          nullptr, c->out_norm, c->model->info.rms_norm_epsilon, xtmp,
                                          xtmp + ((std::max(c->hidden, c->ffn) + 63) / 64 * 64), nullptr);
        te_hip::prof_mark(nullptr, te_hip::kProfLmHead);
        if (s != TE_STATUS_OK) {
            return s;
        }
        if (c->sws == nullptr) {
            c->sws_bytes = te_hip_sample_workspace_bytes(c->vocab);
            unsigned char *p = nullptr;
            if ((s = dev_alloc(c, &p, c->sws_bytes)) != TE_STATUS_OK) {
                return s;
            }
            c->sws = p;
        }
        return te_hip_sample_top_k_f32(c->logits, c->vocab, sm.top_k, sm.temperature, &sm.rng, &id, c->sws,
                                       c->sws_bytes, nullptr);
    }
    return hipMemcpy(&id, c->token, sizeof(id), hipMemcpyDeviceToHost) == hipSuccess ? TE_STATUS_OK
                                                                                   : TE_STATUS_RUNTIME_ERROR;
}

bool stop_token(const te_model *m, uint32_t id) {
    const char *e = getenv("TINYENGINE_IGNORE_EOS");
    if (e != nullptr && e[0] == '1') {
        return false;
    }
    return id == m->tok.eos_token_id || id == m->tok.padding_token_id;
}

te_status emit(const te_model *m, uint32_t id, te_token_callback cb, void *ud) {
    if (cb == nullptr) {
        return TE_STATUS_OK;
    }
    std::string text;
    const te_status s = detokenize(m, &id, 1, 1, text);
    if (s == TE_STATUS_OK) {
        cb(text.c_str(), id, ud);
    }
    return s;
}

// te_qwen_generate_text (qwen.c:260-400) on the GPU.
// TINYENGINE_PROFILE (set, not "0"): one line on stderr per generate call in
// the reference's format (qwen.c:2262-2304: total, tokenize, init and
// embedding times, then each matvec bucket as ms/calls), followed by this
// build's attention and elementwise buckets and the prompt / generation
// split.  GPU buckets are HIP-event times of the launches (te_hip::prof_*);
// total, tokenize, init, prefill and decode are wall-clock.
struct ProfileReport {
    typedef std::chrono::steady_clock clock;
    bool on = false;
    clock::time_point t0 = clock::now(), mark = t0;
    double tokenize_ms = 0.0, init_ms = 0.0, prefill_ms = 0.0, decode_ms = 0.0;
    size_t prompt_tokens = 0;
    uint32_t generated = 0;
    ProfileReport() {
        const char *e = getenv("TINYENGINE_PROFILE");
        on = e != nullptr && strcmp(e, "0") != 0;
        if (on) {
            te_hip::prof_start();
        }
    }
    double lap() {  // ms since the previous lap
        const clock::time_point t = clock::now();
        const double ms = std::chrono::duration<double, std::milli>(t - mark).count();
        mark = t;
        return ms;
    }
    ~ProfileReport() {
        if (!on) {
            return;
        }
        (void)te_hip::prof_flush();
        const double total = std::chrono::duration<double, std::milli>(clock::now() - t0).count();
        using namespace te_hip;
        double matvec = 0.0;
        for (ProfPhase p : {kProfQ, kProfK, kProfV, kProfO, kProfGate, kProfUp, kProfDown, kProfLmHead, kProfOther}) {
            matvec += prof_ms(p);
        }
        auto b = [](ProfPhase p) { return std::make_pair(prof_ms(p), prof_calls(p)); };
        const auto q = b(kProfQ), k = b(kProfK), v = b(kProfV), o = b(kProfO), g = b(kProfGate), u = b(kProfUp),
                   d = b(kProfDown), h = b(kProfLmHead), x = b(kProfOther), at = b(kProfAttention),
                   ew = b(kProfElementwise);
        fprintf(stderr,
                "tinyengine_profile: total_ms=%.2f tokenize_ms=%.2f init_ms=%.2f embed_ms=%.2f matvec_ms=%.2f "
                "q=%.2f/%llu k=%.2f/%llu v=%.2f/%llu o=%.2f/%llu gate=%.2f/%llu up=%.2f/%llu "
                "down=%.2f/%llu lm_head=%.2f/%llu other=%.2f/%llu attention=%.2f/%llu elementwise=%.2f/%llu "
                "prefill_ms=%.2f decode_ms=%.2f prompt_tokens=%zu generated_tokens=%u\n",
                total, tokenize_ms, init_ms, prof_ms(kProfEmbed), matvec, q.first, q.second, k.first, k.second,
                v.first, v.second, o.first, o.second, g.first, g.second, u.first, u.second, d.first, d.second,
                h.first, h.second, x.first, x.second, at.first, at.second, ew.first, ew.second, prefill_ms,
                decode_ms, prompt_tokens, generated);
        prof_stop();
    }
};

te_status generate(te_context *c, const char *prompt, uint32_t max_tokens, te_token_callback cb, void *ud,
                   bool chat) {
    ProfileReport prof;
    te_model *m = c->model;
    std::string text;
    if (chat) {
        text = std::string("<|im_start|>user\n") + prompt + "<|im_end|>\n<|im_start|>assistant\n";
    } else {
        text = prompt;
        if (text.empty()) {
            return TE_STATUS_INVALID_ARGUMENT;
        }
    }
    if (m->tokens.empty()) {
        return TE_STATUS_UNSUPPORTED;
    }
    std::vector<uint32_t> ids;
    te_status s = tokenize(m, text.c_str(), 1, ids);
    if (s != TE_STATUS_OK || ids.empty()) {
        return s == TE_STATUS_OK ? TE_STATUS_RUNTIME_ERROR : s;
    }
    prof.tokenize_ms = prof.lap();
    prof.prompt_tokens = ids.size();
    std::lock_guard<std::mutex> lock(c->mutex);
    if ((s = check_shapes(c, ids.size() + (size_t)max_tokens)) != TE_STATUS_OK) {
        return s;
    }
    if (!c->ready) {
        if ((s = init_state(c)) != TE_STATUS_OK) {
            release_state(c);
            return s;
        }
    }
    prof.init_ms = prof.lap();
    Sampler sm;
    const bool greedy = sm.temperature <= 0.0f;
    // Cache reuse across calls on one context: the positions whose tokens
    // equal the previous call's (prompt and forwarded generated tokens) keep
    // their K / V, as the previous call computed them.  With one numeric path
    // (TINYENGINE_BATCH_PREFILL=0) that is exactly what a fresh context would
    // compute; with the batched prefill, positions the decode path filled
    // (generated tokens) differ from a fresh context's batched values by
    // rounding only.  The last prompt token is always run, for its logits.
    // TINYENGINE_KV_REUSE=0 turns reuse off.
    size_t start = 0;
    const char *reuse = getenv("TINYENGINE_KV_REUSE");
    if (reuse == nullptr || strcmp(reuse, "0") != 0) {
        while (start + 1 < ids.size() && start < c->history.size() && c->history[start] == ids[start]) {
            ++start;
        }
    }
    c->history.resize(start);
    c->vt_valid = std::min(c->vt_valid, start);
    // several new prompt tokens go through the batched prefill unless
    // TINYENGINE_BATCH_PREFILL=0 (the reference's switch, qwen.c:346-347)
    const char *bp = getenv("TINYENGINE_BATCH_PREFILL");
    bool batched = false;
    if (c->batch_ok && ids.size() - start > 1 && (bp == nullptr || strcmp(bp, "0") != 0)) {
        s = prefill_batch(c, ids.data(), start, ids.size());
        if (s == TE_STATUS_OK && greedy) {
            s = project_greedy(c);
        }
        // UNSUPPORTED (a shape the batched kernels do not take): one token at
        // a time instead, as the reference falls back (qwen.c:348-356)
        if (s != TE_STATUS_OK && s != TE_STATUS_UNSUPPORTED) {
            c->history.clear();
            return s;
        }
        batched = s == TE_STATUS_OK;
        if (batched) {
            c->history.insert(c->history.end(), ids.begin() + start, ids.end());
        }
    }
    if (!batched) {
        c->vt_valid = std::min(c->vt_valid, start);  // the per-token path appends to the value cache only
        for (size_t i = start; i < ids.size(); ++i) {
            if ((s = forward(c, ids[i], i, greedy && i + 1 == ids.size())) != TE_STATUS_OK) {
                c->history.clear();
                return s;
            }
            c->history.push_back(ids[i]);
        }
    }
    uint32_t next = 0;
    if ((s = next_token(c, sm, next)) != TE_STATUS_OK) {
        c->history.clear();
        return s;
    }
    if (prof.on) {
        (void)te_hip::prof_flush();
        prof.prefill_ms = prof.lap();
    }
    size_t position = ids.size();
    for (uint32_t g = 0; g < max_tokens; ++g) {
        if (stop_token(m, next)) {
            break;
        }
        if ((s = emit(m, next, cb, ud)) != TE_STATUS_OK) {
            return s;
        }
        ++prof.generated;
        if (g + 1 == max_tokens) {
            break;
        }
        if ((s = forward(c, next, position, greedy)) != TE_STATUS_OK) {
            c->history.clear();
            return s;
        }
        c->history.push_back(next);
        if ((s = next_token(c, sm, next)) != TE_STATUS_OK) {
            return s;
        }
        if (prof.on) {
            (void)te_hip::prof_flush();  // one token's marks at a time
        }
        ++position;
    }
    if (prof.on) {
        prof.decode_ms = prof.lap();
    }
    return TE_STATUS_OK;
}

}  // namespace

extern "C" te_status te_context_create(te_model *model, const te_runtime_options *options, te_context **out_context) {
    if (model == nullptr || out_context == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    te_context *c = new (std::nothrow) te_context();
    if (c == nullptr) {
        return TE_STATUS_OUT_OF_MEMORY;
    }
    c->model = model;
    c->options = options != nullptr ? *options : model->options;
    *out_context = c;
    return TE_STATUS_OK;
}

extern "C" void te_context_free(te_context *context) {
    if (context == nullptr) {
        return;
    }
    release_state(context);
    delete context;
}

// With TINYENGINE_GENERATION=stub the reference's fixed four-piece reply is
// streamed (tinyengine.c:410-423); otherwise the chat-templated generation.
extern "C" te_status te_generate(te_context *context, const char *prompt, uint32_t max_tokens,
                                 te_token_callback callback, void *userdata) {
    if (context == nullptr || prompt == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (max_tokens == 0u) {
        return TE_STATUS_OK;
    }
    const char *mode = getenv("TINYENGINE_GENERATION");
    if (mode != nullptr && strcmp(mode, "stub") == 0) {
        static const char *const pieces[] = {"Mi", " ch", "iamo", " Alex"};
        static const uint32_t ids[] = {41887u, 521u, 34214u, 8515u};
        const uint32_t count = max_tokens < 4u ? max_tokens : 4u;
        for (uint32_t i = 0; i < count; ++i) {
            if (callback != nullptr) {
                callback(pieces[i], ids[i], userdata);
            }
        }
        return TE_STATUS_OK;
    }
    if (context->model == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    try {
        return generate(context, prompt, max_tokens, callback, userdata, true);
    } catch (const std::bad_alloc &) {
        return TE_STATUS_OUT_OF_MEMORY;
    }
}

extern "C" te_status te_generate_raw(te_context *context, const char *prompt, uint32_t max_tokens,
                                     te_token_callback callback, void *userdata) {
    if (context == nullptr || prompt == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (max_tokens == 0u) {
        return TE_STATUS_OK;
    }
    if (context->model == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    try {
        return generate(context, prompt, max_tokens, callback, userdata, false);
    } catch (const std::bad_alloc &) {
        return TE_STATUS_OUT_OF_MEMORY;
    }
}
