// gguf.hip — the model file: a GGUF v1-v3 reader and the qwen35 model load.
//
// Host code only.  The reader follows the GGUF layout (little-endian: magic,
// version, tensor and metadata counts, typed metadata, tensor directory, then
// a data section at the next alignment boundary) with the checks the
// reference's reader makes (crates/codpiece-gguf/src/lib.rs:345-458): count
// and length caps, a power-of-two alignment, tensor offsets aligned, in file
// order without overlap, and inside the data section.  The model load is
// Weights::load (crates/codpiece-model/src/lib.rs:128-311) on one device:
// every tensor's bytes are read from the file and handed to
// cpv_model_set_tensor by name, after the hyper-parameters are taken from the
// metadata as Hparams::from_gguf does (crates/codpiece-model/src/qwen35.rs:
// 75-130).
#include <stdio.h>
#include <string.h>

#include <map>
#include <string>
#include <vector>

#include "cpv_internal.h"

namespace {

constexpr uint32_t MAGIC = 0x46554747u;           // "GGUF"
constexpr uint64_t MAX_TENSORS = 1ull << 20, MAX_KVS = 1ull << 20;
constexpr uint64_t MAX_STRING = 256ull << 20, MAX_ARRAY = 256ull << 20;
constexpr uint32_t MAX_DIMS = 8;

// elements and bytes per block of the ggml types a file may hold (0: unknown)
struct TypeSize { int64_t block, bytes; };
TypeSize type_size(uint32_t t)
{
    switch (t) {
    case 0: return {1, 4};        // F32
    case 1: return {1, 2};        // F16
    case 2: return {32, 18};      // Q4_0
    case 3: return {32, 20};      // Q4_1
    case 6: return {32, 22};      // Q5_0
    case 7: return {32, 24};      // Q5_1
    case 8: return {32, 34};      // Q8_0
    case 9: return {32, 36};      // Q8_1
    case 10: return {256, 84};    // Q2_K
    case 11: return {256, 110};   // Q3_K
    case 12: return {256, 144};   // Q4_K
    case 13: return {256, 176};   // Q5_K
    case 14: return {256, 210};   // Q6_K
    case 15: return {256, 292};   // Q8_K
    case 16: return {256, 66};    // IQ2_XXS
    case 17: return {256, 74};    // IQ2_XS
    case 18: return {256, 98};    // IQ3_XXS
    case 19: return {256, 50};    // IQ1_S
    case 20: return {32, 18};     // IQ4_NL
    case 21: return {256, 110};   // IQ3_S
    case 22: return {256, 82};    // IQ2_S
    case 23: return {256, 136};   // IQ4_XS
    case 24: return {1, 1};       // I8
    case 25: return {1, 2};       // I16
    case 26: return {1, 4};       // I32
    case 27: return {1, 8};       // I64
    case 28: return {1, 8};       // F64
    case 29: return {256, 56};    // IQ1_M
    case 30: return {1, 2};       // BF16
    case 34: return {256, 54};    // TQ1_0
    case 35: return {256, 66};    // TQ2_0
    case 39: return {32, 17};     // MXFP4
    default: return {0, 0};
    }
}

// a metadata value: numbers as u64 / i64 / f64, strings, and arrays (kept as
// their element type and length, plus the values of short numeric arrays)
struct Value {
    uint32_t type = 0;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    bool is_int = false, is_float = false;
    std::string s;
    uint32_t elem = 0;
    uint64_t len = 0;
    std::vector<Value> items;

    bool as_u64(uint64_t* out) const
    {
        if (is_int && i >= 0) { *out = (uint64_t)i; return true; }
        if (type == 4 || type == 10 || type == 0 || type == 2) { *out = u; return true; }
        return false;
    }
    bool as_f64(double* out) const
    {
        if (is_float) { *out = f; return true; }
        uint64_t v;
        if (as_u64(&v)) { *out = (double)v; return true; }
        return false;
    }
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
    int64_t bytes = -1;      // -1: a type without a known size
};

struct File {
    uint32_t version = 0;
    uint64_t alignment = 32, data_start = 0, file_len = 0;
    std::map<std::string, Value> kvs;
    std::vector<Tensor> tensors;
};

struct Reader {
    FILE* f;
    bool wide = true;        // counts and lengths are u64 from version 3, u32 before
    std::string* err;

    bool bytes(void* p, size_t n)
    {
        if (fread(p, 1, n, f) != n) { *err = "unexpected end of file"; return false; }
        return true;
    }
    template <class T>
    bool num(T* v) { return bytes(v, sizeof(T)); }
    bool len(uint64_t* v)
    {
        if (wide) return num(v);
        uint32_t w;
        if (!num(&w)) return false;
        *v = w;
        return true;
    }
    bool str(std::string* s)
    {
        uint64_t n;
        if (!len(&n)) return false;
        if (n > MAX_STRING) { *err = "string length " + std::to_string(n) + " exceeds the cap"; return false; }
        s->resize(n);
        return n == 0 || bytes(&(*s)[0], n);
    }
    bool value(uint32_t type, int depth, Value* v, bool keep)
    {
        v->type = type;
        switch (type) {
        case 0: { uint8_t x; if (!num(&x)) return false; v->u = x; v->i = x; v->is_int = true; return true; }
        case 1: { int8_t x; if (!num(&x)) return false; v->i = x; v->is_int = true; return true; }
        case 2: { uint16_t x; if (!num(&x)) return false; v->u = x; v->i = x; v->is_int = true; return true; }
        case 3: { int16_t x; if (!num(&x)) return false; v->i = x; v->is_int = true; return true; }
        case 4: { uint32_t x; if (!num(&x)) return false; v->u = x; v->i = x; v->is_int = true; return true; }
        case 5: { int32_t x; if (!num(&x)) return false; v->i = x; v->is_int = true; return true; }
        case 6: { float x; if (!num(&x)) return false; v->f = x; v->is_float = true; return true; }
        case 7: { uint8_t x; if (!num(&x)) return false; v->u = x != 0; return true; }
        case 8: return str(&v->s);
        case 9: {
            if (depth > 2) { *err = "array nesting too deep"; return false; }
            if (!num(&v->elem) || !len(&v->len)) return false;
            if (v->len > MAX_ARRAY) { *err = "array length " + std::to_string(v->len) + " exceeds the cap"; return false; }
            // short arrays of numbers are kept (rope sections); the rest are walked
            const bool keep_items = keep && v->len <= 64 && v->elem != 8 && v->elem != 9;
            for (uint64_t k = 0; k < v->len; k++) {
                Value e;
                if (!value(v->elem, depth + 1, &e, false)) return false;
                if (keep_items) v->items.push_back(e);
            }
            return true;
        }
        case 10: { uint64_t x; if (!num(&x)) return false; v->u = x; v->i = (int64_t)x; v->is_int = x <= INT64_MAX; return true; }
        case 11: { int64_t x; if (!num(&x)) return false; v->i = x; v->is_int = true; return true; }
        case 12: { double x; if (!num(&x)) return false; v->f = x; v->is_float = true; return true; }
        default: *err = "unknown metadata value type " + std::to_string(type); return false;
        }
    }
};

bool open_file(const char* path, File* g, std::string* err)
{
    FILE* f = fopen(path, "rb");
    if (!f) { *err = std::string("cannot open ") + path; return false; }
    bool ok = false;
    do {
        if (fseek(f, 0, SEEK_END) != 0) { *err = "cannot seek"; break; }
        const long end = ftell(f);
        if (end < 0 || fseek(f, 0, SEEK_SET) != 0) { *err = "cannot seek"; break; }
        g->file_len = (uint64_t)end;
        Reader r{f, true, err};
        uint32_t magic;
        if (!r.num(&magic)) break;
        if (magic != MAGIC) {
            char b[64];
            snprintf(b, sizeof b, "not a GGUF file: it starts with 0x%08x where the magic 0x%08x belongs", magic, MAGIC);
            *err = b;
            break;
        }
        if (!r.num(&g->version)) break;
        if (g->version < 1 || g->version > 3) { *err = "unsupported GGUF version " + std::to_string(g->version); break; }
        r.wide = g->version >= 3;
        uint64_t nt, nk;
        if (!r.len(&nt) || !r.len(&nk)) break;
        if (nt > MAX_TENSORS || nk > MAX_KVS) {
            *err = "header lists " + std::to_string(nt) + " tensors and " + std::to_string(nk) +
                   " metadata entries, more than this reader accepts (2^20 of each)";
            break;
        }
        bool bad = false;
        for (uint64_t k = 0; k < nk && !bad; k++) {
            std::string key;
            uint32_t type;
            Value v;
            if (!r.str(&key) || !r.num(&type) || !r.value(type, 0, &v, true)) { bad = true; break; }
            g->kvs[key] = v;
        }
        if (bad) break;
        auto al = g->kvs.find("general.alignment");
        if (al != g->kvs.end()) {
            uint64_t a = 0;
            if (!al->second.as_u64(&a)) a = 0;
            g->alignment = a;
        }
        if (g->alignment == 0 || (g->alignment & (g->alignment - 1))) {
            *err = "bad alignment " + std::to_string(g->alignment);
            break;
        }
        g->tensors.resize(nt);
        for (uint64_t k = 0; k < nt && !bad; k++) {
            Tensor& t = g->tensors[k];
            uint32_t nd;
            if (!r.str(&t.name) || !r.num(&nd)) { bad = true; break; }
            if (nd > MAX_DIMS) { *err = "tensor " + t.name + ": " + std::to_string(nd) + " dims"; bad = true; break; }
            t.dims.resize(nd);
            for (uint32_t d = 0; d < nd && !bad; d++) bad = !r.len(&t.dims[d]);
            if (bad || !r.num(&t.type) || !r.num(&t.offset)) { bad = true; break; }
            const TypeSize ts = type_size(t.type);
            if (ts.block > 0) {
                // elements, then blocks of the row-padded ggml layout (the row length is a whole number of blocks)
                uint64_t n = 1;
                for (uint64_t d : t.dims) {
                    if (d && n > UINT64_MAX / d) { *err = "tensor " + t.name + ": element count overflows"; bad = true; break; }
                    n *= d;
                }
                if (bad) break;
                if (n % (uint64_t)ts.block) { *err = "tensor " + t.name + ": not a whole number of blocks"; bad = true; break; }
                t.bytes = (int64_t)(n / (uint64_t)ts.block * (uint64_t)ts.bytes);
            }
        }
        if (bad) break;
        const long pos = ftell(f);
        if (pos < 0) { *err = "cannot tell"; break; }
        g->data_start = ((uint64_t)pos + g->alignment - 1) / g->alignment * g->alignment;
        // the directory's tensors in the data section: aligned, in order, inside the file
        if (g->data_start > g->file_len) { *err = "data section starts past the end of the file"; break; }
        const uint64_t data_len = g->file_len - g->data_start;
        uint64_t prev_end = 0;
        for (const Tensor& t : g->tensors) {
            if (t.offset % g->alignment) { *err = "tensor " + t.name + " offset not aligned"; bad = true; break; }
            if (t.offset < prev_end) { *err = "tensor " + t.name + " overlaps the previous one"; bad = true; break; }
            if (t.bytes >= 0) {
                const uint64_t end = t.offset + (uint64_t)t.bytes;
                if (end < t.offset || end > data_len) {
                    *err = "tensor " + t.name + " would end at byte " + std::to_string(end) +
                           " of a data section that holds " + std::to_string(data_len);
                    bad = true;
                    break;
                }
                prev_end = end;
            } else {
                prev_end = t.offset;
            }
        }
        if (bad) break;
        ok = true;
    } while (false);
    fclose(f);
    return ok;
}

void put_err(char* buf, int len, const std::string& msg)
{
    if (buf && len > 0) snprintf(buf, (size_t)len, "%s", msg.c_str());
}

// Hparams::from_gguf for the all-attention qwen35 layout
cpv_status hparams_of(const File& g, cpv_hparams* hp, std::string* err)
{
    auto kv = [&](const std::string& k) -> const Value* {
        auto it = g.kvs.find(k);
        return it == g.kvs.end() ? nullptr : &it->second;
    };
    const Value* arch = kv("general.architecture");
    if (!arch || arch->type != 8) { *err = "no architecture"; return CPV_EINVAL; }
    if (arch->s != "qwen35") { *err = "architecture \"" + arch->s + "\", want qwen35"; return CPV_EUNSUPPORTED; }
    auto u = [&](const char* key, uint64_t* out) {
        const Value* v = kv(std::string("qwen35.") + key);
        return v && v->as_u64(out);
    };
    auto fl = [&](const char* key, double* out) {
        const Value* v = kv(std::string("qwen35.") + key);
        return v && v->as_f64(out);
    };
    uint64_t blocks, embd, heads, heads_kv, ff;
    const char* missing = nullptr;
    if (!u("block_count", &blocks)) missing = "block_count";
    else if (!u("embedding_length", &embd)) missing = "embedding_length";
    else if (!u("attention.head_count", &heads)) missing = "attention.head_count";
    else if (!u("attention.head_count_kv", &heads_kv)) missing = "attention.head_count_kv";
    else if (!u("feed_forward_length", &ff)) missing = "feed_forward_length";
    if (missing) { *err = std::string("missing qwen35.") + missing; return CPV_EINVAL; }
    uint64_t nextn = 0, head_k = heads ? embd / heads : 0, head_v, n_rot, interval = 4;
    u("nextn_predict_layers", &nextn);
    u("attention.key_length", &head_k);
    head_v = head_k;
    u("attention.value_length", &head_v);
    n_rot = head_k;
    u("rope.dimension_count", &n_rot);
    u("full_attention_interval", &interval);
    double eps = 1e-6, base = 10000.0;
    fl("attention.layer_norm_rms_epsilon", &eps);
    fl("rope.freq_base", &base);
    const Value* tok = kv("tokenizer.ggml.tokens");
    if (!tok || tok->type != 9) { *err = "missing tokenizer tokens"; return CPV_EINVAL; }
    if (interval != 1) {
        *err = "full_attention_interval " + std::to_string(interval) + ": recurrent (GDN) layers are not supported";
        return CPV_EUNSUPPORTED;
    }
    if (nextn > 1 || nextn >= blocks) { *err = std::to_string(nextn) + " nextn layers"; return CPV_EUNSUPPORTED; }
    if (head_v != head_k) { *err = "value length differs from key length"; return CPV_EUNSUPPORTED; }
    if (embd > INT32_MAX || heads > INT32_MAX || heads_kv > INT32_MAX || head_k > INT32_MAX || ff > INT32_MAX ||
        tok->len > INT32_MAX || n_rot > INT32_MAX || blocks > INT32_MAX) {
        *err = "hyper-parameter out of range";
        return CPV_EINVAL;
    }
    memset(hp, 0, sizeof *hp);
    hp->n_layer = (int32_t)(blocks - nextn);
    hp->n_embd = (int32_t)embd;
    hp->n_head = (int32_t)heads;
    hp->n_head_kv = (int32_t)heads_kv;
    hp->head_dim = (int32_t)head_k;
    hp->n_ff = (int32_t)ff;
    hp->n_vocab = (int32_t)tok->len;
    hp->n_rot = (int32_t)n_rot;
    const Value* sec = kv("qwen35.rope.dimension_sections");
    if (sec && sec->type == 9)
        for (size_t k = 0; k < sec->items.size() && k < 4; k++) {
            uint64_t v = 0;
            if (sec->items[k].as_u64(&v)) hp->rope_sections[k] = (int32_t)v;
        }
    hp->rms_eps = (float)eps;
    hp->freq_base = (float)base;
    hp->has_mtp = nextn > 0;
    return CPV_OK;
}

}  // namespace

extern "C" cpv_status cpv_gguf_scan(const char* path, cpv_gguf_info* info, char* errbuf, int errlen)
{
    if (!path || !info) { put_err(errbuf, errlen, "gguf_scan: null argument"); return CPV_EINVAL; }
    File g;
    std::string err;
    if (!open_file(path, &g, &err)) { put_err(errbuf, errlen, err); return CPV_EINVAL; }
    info->version = (int32_t)g.version;
    info->n_tensors = (int64_t)g.tensors.size();
    info->n_kv = (int64_t)g.kvs.size();
    info->alignment = g.alignment;
    info->data_start = g.data_start;
    uint64_t tb = 0;
    for (const Tensor& t : g.tensors)
        if (t.bytes > 0) tb += (uint64_t)t.bytes;
    info->tensor_bytes = tb;
    return CPV_OK;
}

extern "C" cpv_status cpv_gguf_hparams(const char* path, cpv_hparams* hp, char* errbuf, int errlen)
{
    if (!path || !hp) { put_err(errbuf, errlen, "gguf_hparams: null argument"); return CPV_EINVAL; }
    File g;
    std::string err;
    if (!open_file(path, &g, &err)) { put_err(errbuf, errlen, err); return CPV_EINVAL; }
    const cpv_status st = hparams_of(g, hp, &err);
    if (st != CPV_OK) put_err(errbuf, errlen, err);
    return st;
}

extern "C" cpv_status cpv_model_load_gguf(cpv_ctx* ctx, const char* path, cpv_model** out)
{
    if (!ctx || !path || !out) return cpv_fail(ctx, CPV_EINVAL, "load_gguf: null argument");
    *out = nullptr;
    File g;
    std::string err;
    if (!open_file(path, &g, &err)) return cpv_fail(ctx, CPV_EINVAL, "load_gguf: %s", err.c_str());
    cpv_hparams hp;
    cpv_status st = hparams_of(g, &hp, &err);
    if (st != CPV_OK) return cpv_fail(ctx, st, "load_gguf: %s", err.c_str());
    // every tensor's shape and type first, so that nothing is read for a file the model cannot take
    size_t most = 0;
    for (const Tensor& t : g.tensors) {
        if (t.bytes < 0) return cpv_fail(ctx, CPV_EUNSUPPORTED, "load_gguf: %s has type %u", t.name.c_str(), t.type);
        for (size_t d = 2; d < t.dims.size(); d++)
            if (t.dims[d] != 1)
                return cpv_fail(ctx, CPV_EUNSUPPORTED, "load_gguf: %s has more than two dimensions", t.name.c_str());
        if (t.dims.empty() || t.dims[0] > INT64_MAX || (t.dims.size() > 1 && t.dims[1] > INT64_MAX))
            return cpv_fail(ctx, CPV_EINVAL, "load_gguf: %s has a bad shape", t.name.c_str());
        most = (size_t)t.bytes > most ? (size_t)t.bytes : most;
    }
    cpv_model* m = nullptr;
    if ((st = cpv_model_create(ctx, &hp, &m)) != CPV_OK) return st;
    std::vector<uint8_t> buf(most ? most : 1);
    FILE* f = fopen(path, "rb");
    if (!f) {
        cpv_model_free(m);
        return cpv_fail(ctx, CPV_EINVAL, "load_gguf: cannot open %s", path);
    }
    // one whole-tensor read and one upload per tensor, in file order
    for (const Tensor& t : g.tensors) {
        const uint64_t at = g.data_start + t.offset;
        if (fseeko(f, (off_t)at, SEEK_SET) != 0 || fread(buf.data(), 1, (size_t)t.bytes, f) != (size_t)t.bytes) {
            fclose(f);
            cpv_model_free(m);
            return cpv_fail(ctx, CPV_EINVAL, "load_gguf: cannot read %s", t.name.c_str());
        }
        const int64_t ne0 = (int64_t)t.dims[0], ne1 = t.dims.size() > 1 ? (int64_t)t.dims[1] : 1;
        if ((st = cpv_model_set_tensor(m, t.name.c_str(), (int)t.type, buf.data(), 0, ne0, ne1)) != CPV_OK) {
            fclose(f);
            cpv_model_free(m);
            return st;
        }
    }
    fclose(f);
    if ((st = cpv_model_ready(m)) != CPV_OK) {
        cpv_model_free(m);
        return st;
    }
    *out = m;
    return CPV_OK;
}
