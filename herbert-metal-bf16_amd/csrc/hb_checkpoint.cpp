// hb_checkpoint.cpp -- the checkpoint read in place: safetensors shards
// mapped read-only, tensor names normalised to the engine's keys, and the
// matmul path's weights uploaded in the fused layouts the kernels read
// ([q | k | v] rows, [gate | up] rows), each element rounded once to bf16
// from its stored type.
//
// Reference: src/model/qwen.rs:155-375 (Checkpoint::load: the index's
// shards, the mapping, `normalize` :102-153, `bf16` / `read_bf16_into`
// :301-361, bf16_at :92-99) and the uploads of QwenEngine::load
// (src/metal/qwen.rs:776-835: `upload(&mut gpu, &ck, &[(name, len), ...])`
// stacks its parts' rows into one buffer).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "hb_internal.h"

namespace {

// ---- a small JSON reader: the safetensors header and the shard index ----
struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    double num = 0;
    bool b = false;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json* get(const std::string& k) const {
        for (const auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct Parser {
    const char* p;
    const char* end;
    std::string err;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool lit(const char* s) {
        size_t n = strlen(s);
        if ((size_t)(end - p) < n || memcmp(p, s, n)) return false;
        p += n;
        return true;
    }
    bool string(std::string* out) {
        if (p >= end || *p != '"') return fail("string expected");
        p++;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                if (++p >= end) return fail("bad escape");
                char c = *p++;
                switch (c) {
                    case 'n': *out += '\n'; break;
                    case 't': *out += '\t'; break;
                    case 'r': *out += '\r'; break;
                    case 'b': *out += '\b'; break;
                    case 'f': *out += '\f'; break;
                    case 'u': {
                        if (end - p < 4) return fail("bad \\u escape");
                        unsigned v = 0;
                        for (int i = 0; i < 4; i++) {
                            char h = *p++;
                            v <<= 4;
                            if (h >= '0' && h <= '9') v |= h - '0';
                            else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
                            else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
                            else return fail("bad \\u escape");
                        }
                        // UTF-8 of the code unit (names are ASCII in practice).
                        if (v < 0x80) *out += (char)v;
                        else if (v < 0x800) *out += (char)(0xC0 | (v >> 6)), *out += (char)(0x80 | (v & 0x3F));
                        else *out += (char)(0xE0 | (v >> 12)), *out += (char)(0x80 | ((v >> 6) & 0x3F)),
                                 *out += (char)(0x80 | (v & 0x3F));
                        break;
                    }
                    default: *out += c;
                }
            } else {
                *out += *p++;
            }
        }
        if (p >= end) return fail("unterminated string");
        p++;
        return true;
    }
    bool fail(const char* m) {
        if (err.empty()) err = m;
        return false;
    }
    bool value(Json* v, int depth = 0) {
        if (depth > 32) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("value expected");
        if (*p == '{') {
            v->kind = Json::Obj;
            p++;
            ws();
            if (p < end && *p == '}') return p++, true;
            for (;;) {
                std::string k;
                ws();
                if (!string(&k)) return false;
                ws();
                if (p >= end || *p != ':') return fail("':' expected");
                p++;
                v->obj.emplace_back(k, Json());
                if (!value(&v->obj.back().second, depth + 1)) return false;
                ws();
                if (p < end && *p == ',') { p++; continue; }
                if (p < end && *p == '}') return p++, true;
                return fail("',' or '}' expected");
            }
        }
        if (*p == '[') {
            v->kind = Json::Arr;
            p++;
            ws();
            if (p < end && *p == ']') return p++, true;
            for (;;) {
                v->arr.emplace_back();
                if (!value(&v->arr.back(), depth + 1)) return false;
                ws();
                if (p < end && *p == ',') { p++; continue; }
                if (p < end && *p == ']') return p++, true;
                return fail("',' or ']' expected");
            }
        }
        if (*p == '"') {
            v->kind = Json::Str;
            return string(&v->str);
        }
        if (lit("true")) return v->kind = Json::Bool, v->b = true, true;
        if (lit("false")) return v->kind = Json::Bool, v->b = false, true;
        if (lit("null")) return v->kind = Json::Null, true;
        char* e = nullptr;
        std::string tok;
        while (p < end && (strchr("+-.eE", *p) || (*p >= '0' && *p <= '9'))) tok += *p++;
        if (tok.empty()) return fail("unexpected character");
        v->kind = Json::Num;
        v->num = strtod(tok.c_str(), &e);
        if (!e || *e) return fail("bad number");
        return true;
    }
};

bool parse_json(const char* s, size_t n, Json* out, std::string* err) {
    Parser ps{s, s + n, ""};
    if (!ps.value(out)) {
        *err = ps.err;
        return false;
    }
    ps.ws();
    if (ps.p != ps.end) {
        *err = "trailing characters";
        return false;
    }
    return true;
}

enum class Dt { Bf16, F16, F32 };

struct Entry {
    std::vector<uint64_t> shape;
    size_t map;
    uint64_t offset, bytes;
    Dt dt;
    uint64_t elements() const { return bytes / (dt == Dt::F32 ? 4 : 2); }
};

struct Mapping {
    void* base = nullptr;
    size_t size = 0;
};

// The engine's key of a checkpoint name (model/qwen.rs:102-153): the
// prefixes of the Hugging Face layouts dropped, "layers.N.field" -> "N.field";
// the fields of the matmul path and its norms kept, any other one skipped.
bool normalize(const std::string& name, std::string* key) {
    std::string rest = name;
    for (const char* pre : {"language_model.model.", "model.language_model.", "model."})
        if (rest.rfind(pre, 0) == 0) {
            rest = rest.substr(strlen(pre));
            break;
        }
    if (rest == "embed_tokens.weight") return *key = "embed_tokens", true;
    if (rest == "norm.weight") return *key = "norm", true;
    if (rest == "lm_head.weight" || name == "lm_head.weight") return *key = "lm_head", true;
    if (rest.rfind("layers.", 0) != 0) return false;
    rest = rest.substr(7);
    size_t dot = rest.find('.');
    if (dot == std::string::npos || dot == 0) return false;
    for (size_t i = 0; i < dot; i++)
        if (rest[i] < '0' || rest[i] > '9') return false;
    const std::string field = rest.substr(dot + 1);
    static const std::set<std::string> used = {
        "input_layernorm.weight", "post_attention_layernorm.weight",
        "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
        "self_attn.o_proj.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight",
        "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight",
        "mlp.gate.weight", "mlp.experts.gate_up_proj", "mlp.experts.down_proj",
        "mlp.shared_expert.gate_proj.weight", "mlp.shared_expert.up_proj.weight",
        "mlp.shared_expert.down_proj.weight", "mlp.shared_expert_gate.weight",
        "linear_attn.in_proj_qkv.weight", "linear_attn.in_proj_z.weight",
        "linear_attn.in_proj_a.weight", "linear_attn.in_proj_b.weight",
        "linear_attn.out_proj.weight", "linear_attn.norm.weight"};
    if (!used.count(field)) return false;
    *key = std::to_string(strtoul(rest.substr(0, dot).c_str(), nullptr, 10)) + "." + field;
    return true;
}

uint16_t f32_bits_to_bf16(uint32_t b) { return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16); }

// IEEE half to f32, exact.
float f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t b;
    if (e == 0) {
        if (!m) b = s;
        else {  // subnormal: normalise
            int sh = 0;
            while (!(m & 0x400)) m <<= 1, sh++;
            m &= 0x3ff;
            b = s | ((uint32_t)(113 - sh) << 23) | (m << 13);
        }
    } else if (e == 31) {
        b = s | 0x7f800000u | (m << 13);
    } else {
        b = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &b, 4);
    return f;
}

}  // namespace

struct hb_ckpt {
    std::vector<Mapping> maps;
    std::map<std::string, Entry> entries;
    std::string skipped;  // "[loader] skipped: ..." of the reference's log
    ~hb_ckpt() {
        for (auto& m : maps)
            if (m.base) munmap(m.base, m.size);
    }
};

using hb::fail;

static bool read_file(const std::string& path, std::string* out) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return false;
    char buf[65536];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) out->append(buf, n);
    fclose(f);
    return true;
}

// One shard mapped and its tensors entered (the first shard wins a name).
static int add_shard(hb_ckpt* ck, const std::string& path, std::map<std::string, int>* skipped) {
    int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) return fail(HB_ERR_INVALID, path + ": cannot open");
    struct stat st;
    if (fstat(fd, &st) || st.st_size < 8) {
        close(fd);
        return fail(HB_ERR_INVALID, path + ": not a safetensors file (too short)");
    }
    void* base = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (base == MAP_FAILED) return fail(HB_ERR_INVALID, path + ": mmap failed");
    ck->maps.push_back({base, (size_t)st.st_size});
    const size_t map = ck->maps.size() - 1;
    const unsigned char* b = (const unsigned char*)base;
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | b[i];
    if (hlen > (uint64_t)st.st_size - 8) return fail(HB_ERR_INVALID, path + ": header runs past the file");
    Json h;
    std::string err;
    if (!parse_json((const char*)b + 8, (size_t)hlen, &h, &err) || h.kind != Json::Obj)
        return fail(HB_ERR_INVALID, path + ": bad header: " + err);
    const uint64_t data0 = 8 + hlen, data_len = (uint64_t)st.st_size - data0;
    for (const auto& kv : h.obj) {
        if (kv.first == "__metadata__") continue;
        std::string key;
        if (!normalize(kv.first, &key)) {
            size_t d1 = kv.first.find('.'), d2 = d1 == std::string::npos ? d1 : kv.first.find('.', d1 + 1);
            (*skipped)[kv.first.substr(0, d2)]++;
            continue;
        }
        const Json* dt = kv.second.get("dtype");
        const Json* shape = kv.second.get("shape");
        const Json* off = kv.second.get("data_offsets");
        if (!dt || dt->kind != Json::Str || !shape || shape->kind != Json::Arr || !off ||
            off->kind != Json::Arr || off->arr.size() != 2)
            return fail(HB_ERR_INVALID, path + ": " + kv.first + ": bad entry");
        Entry e;
        if (dt->str == "BF16") e.dt = Dt::Bf16;
        else if (dt->str == "F16") e.dt = Dt::F16;
        else if (dt->str == "F32") e.dt = Dt::F32;
        else return fail(HB_ERR_INVALID, "unsupported dtype " + dt->str + " for " + kv.first);
        uint64_t count = 1;
        for (const auto& s : shape->arr) {
            if (s.kind != Json::Num || s.num < 0) return fail(HB_ERR_INVALID, kv.first + ": bad shape");
            e.shape.push_back((uint64_t)s.num);
            count *= (uint64_t)s.num;
        }
        const uint64_t s0 = (uint64_t)off->arr[0].num, s1 = (uint64_t)off->arr[1].num;
        if (s1 < s0 || s1 > data_len) return fail(HB_ERR_INVALID, path + ": " + kv.first + ": offsets past the data");
        e.map = map;
        e.offset = data0 + s0;
        e.bytes = s1 - s0;
        if (e.elements() != count || e.bytes % (e.dt == Dt::F32 ? 4 : 2))
            return fail(HB_ERR_INVALID, kv.first + ": shape and byte size disagree");
        ck->entries.emplace(key, e);  // the shards win where both have a name
    }
    return HB_OK;
}

extern "C" {

int hb_ckpt_open(const char* dir, hb_ckpt** out) {
    *out = nullptr;
    std::unique_ptr<hb_ckpt> ck(new hb_ckpt);
    const std::string d = dir;
    std::vector<std::string> shards;
    std::string idx;
    if (read_file(d + "/model.safetensors.index.json", &idx)) {
        Json j;
        std::string err;
        if (!parse_json(idx.data(), idx.size(), &j, &err) || !j.get("weight_map") ||
            j.get("weight_map")->kind != Json::Obj)
            return fail(HB_ERR_INVALID, d + "/model.safetensors.index.json: no weight_map (" + err + ")");
        std::set<std::string> set;
        for (const auto& kv : j.get("weight_map")->obj)
            if (kv.second.kind == Json::Str) set.insert(kv.second.str);
        shards.assign(set.begin(), set.end());  // sorted, as the reference's
    } else {
        shards.push_back("model.safetensors");
    }
    std::map<std::string, int> skipped;
    for (const auto& s : shards) {
        int rc = add_shard(ck.get(), d + "/" + s, &skipped);
        if (rc) return rc;
    }
    for (const auto& kv : skipped)
        ck->skipped += (ck->skipped.empty() ? "" : ", ") + kv.first + ".* x" + std::to_string(kv.second);
    *out = ck.release();
    return HB_OK;
}

void hb_ckpt_close(hb_ckpt* ck) { delete ck; }

const char* hb_ckpt_skipped(hb_ckpt* ck) { return ck ? ck->skipped.c_str() : ""; }

uint64_t hb_ckpt_elements(hb_ckpt* ck, const char* key) {
    auto it = ck->entries.find(key);
    return it == ck->entries.end() ? 0 : it->second.elements();
}

// The parts (key, elements) one after the other as bf16 into dst (host).
int hb_ckpt_read(hb_ckpt* ck, const char* const* keys, const uint64_t* lens, uint32_t n,
                 uint16_t* dst, uint64_t dst_elements) {
    uint64_t total = 0;
    std::vector<const Entry*> list;
    for (uint32_t i = 0; i < n; i++) {
        auto it = ck->entries.find(keys[i]);
        if (it == ck->entries.end()) return fail(HB_ERR_INVALID, std::string("missing tensor ") + keys[i]);
        if (it->second.elements() != lens[i])
            return fail(HB_ERR_INVALID, std::string(keys[i]) + ": " + std::to_string(it->second.elements()) +
                                            " elements, " + std::to_string(lens[i]) + " expected");
        list.push_back(&it->second);
        total += lens[i];
    }
    if (total > dst_elements)
        return fail(HB_ERR_INVALID, std::to_string(total) + " elements to read into " + std::to_string(dst_elements));
    for (const Entry* e : list) {
        const unsigned char* src = (const unsigned char*)ck->maps[e->map].base + e->offset;
        const uint64_t cnt = e->elements();
        if (e->dt == Dt::Bf16) {
            memcpy(dst, src, cnt * 2);
        } else if (e->dt == Dt::F16) {
            for (uint64_t i = 0; i < cnt; i++) {
                uint16_t h;
                memcpy(&h, src + 2 * i, 2);
                float f = f16_to_f32(h);
                uint32_t bits;
                memcpy(&bits, &f, 4);
                dst[i] = f32_bits_to_bf16(bits);
            }
        } else {
            for (uint64_t i = 0; i < cnt; i++) {
                uint32_t bits;
                memcpy(&bits, src + 4 * i, 4);
                dst[i] = f32_bits_to_bf16(bits);
            }
        }
        dst += cnt;
    }
    return HB_OK;
}

int hb_ckpt_upload(hb_gpu* g, hb_ckpt* ck, const char* const* keys, const uint64_t* lens, uint32_t n,
                   hb_buf* out) {
    uint64_t total = 0;
    for (uint32_t i = 0; i < n; i++) total += lens[i];
    if (!total) return fail(HB_ERR_INVALID, "hb_ckpt_upload: no elements");
    std::vector<uint16_t> host;
    try {
        host.resize(total);
    } catch (...) {
        return fail(HB_ERR_INVALID, "hb_ckpt_upload: host staging of " + std::to_string(total * 2) + " bytes");
    }
    int rc = hb_ckpt_read(ck, keys, lens, n, host.data(), total);
    if (rc) return rc;
    hb_buf b;
    if ((rc = hb_alloc(g, total * 2, &b))) return rc;
    if ((rc = hb_upload(g, b, 0, host.data(), total * 2))) {
        hb_free(g, b);
        return rc;
    }
    *out = b;
    return HB_OK;
}

}  // extern "C"
