// Expert banks on the host: the checkpoint reader of one tensor-parallel rank (safetensors files and their index,
// the split rules, whole tensors cut to the rank's share and pre-sharded stored ranks joined), one layer's routed
// experts loaded into device slabs and tables (the ea_routed the kernels read), and the live change of experts' widths
// with the tables rewritten in place.
//
// Reference: weights.zig:20-240 (Reader: open, openFile, has, get, cut, join), split.zig:7-81 (rules, checkCut,
// share), core/safetensors.zig (header format), moe.zig:65-225 (loadFrom: slabs, ptr / k2 tables, stacked scales,
// codebook marker), expert_swap.zig:301-467 (reader of a width's bank, swapLayer).
#include <fcntl.h>
#include <hip/hip_runtime_api.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "ea_exl3.h"

namespace ea {
namespace bank {

// ---- a small JSON reader: objects, arrays, strings, numbers, true / false / null (the safetensors header and the
// index's weight_map)

struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0;
    bool integral = false;
    uint64_t u = 0;  // exact when integral and non-negative
    std::string s;
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
    bool ok = true;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool lit(const char* w) {
        const size_t n = strlen(w);
        if ((size_t)(end - p) < n || memcmp(p, w, n) != 0) return false;
        p += n;
        return true;
    }
    static void utf8(std::string& o, uint32_t c) {
        if (c < 0x80) o += (char)c;
        else if (c < 0x800) {
            o += (char)(0xC0 | (c >> 6));
            o += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            o += (char)(0xE0 | (c >> 12));
            o += (char)(0x80 | ((c >> 6) & 0x3F));
            o += (char)(0x80 | (c & 0x3F));
        } else {
            o += (char)(0xF0 | (c >> 18));
            o += (char)(0x80 | ((c >> 12) & 0x3F));
            o += (char)(0x80 | ((c >> 6) & 0x3F));
            o += (char)(0x80 | (c & 0x3F));
        }
    }
    bool hex4(uint32_t& v) {
        if (end - p < 4) return false;
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = p[i];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        p += 4;
        return true;
    }
    bool str(std::string& o) {
        if (p >= end || *p != '"') return false;
        ++p;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                if (++p >= end) return false;
                const char c = *p++;
                switch (c) {
                    case '"': o += '"'; break;
                    case '\\': o += '\\'; break;
                    case '/': o += '/'; break;
                    case 'b': o += '\b'; break;
                    case 'f': o += '\f'; break;
                    case 'n': o += '\n'; break;
                    case 'r': o += '\r'; break;
                    case 't': o += '\t'; break;
                    case 'u': {
                        uint32_t v;
                        if (!hex4(v)) return false;
                        if (v >= 0xD800 && v < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                            p += 2;
                            uint32_t lo;
                            if (!hex4(lo)) return false;
                            v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
                        }
                        utf8(o, v);
                        break;
                    }
                    default: return false;
                }
            } else {
                o += *p++;
            }
        }
        if (p >= end) return false;
        ++p;
        return true;
    }
    bool value(Json& v, int depth) {
        if (depth > 64) return false;
        ws();
        if (p >= end) return false;
        const char c = *p;
        if (c == '{') {
            v.kind = Json::OBJ;
            ++p;
            ws();
            if (p < end && *p == '}') {
                ++p;
                return true;
            }
            for (;;) {
                ws();
                std::string k;
                if (!str(k)) return false;
                ws();
                if (p >= end || *p != ':') return false;
                ++p;
                v.obj.emplace_back(std::move(k), Json{});
                if (!value(v.obj.back().second, depth + 1)) return false;
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == '}') {
                    ++p;
                    return true;
                }
                return false;
            }
        }
        if (c == '[') {
            v.kind = Json::ARR;
            ++p;
            ws();
            if (p < end && *p == ']') {
                ++p;
                return true;
            }
            for (;;) {
                v.arr.emplace_back();
                if (!value(v.arr.back(), depth + 1)) return false;
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == ']') {
                    ++p;
                    return true;
                }
                return false;
            }
        }
        if (c == '"') {
            v.kind = Json::STR;
            return str(v.s);
        }
        if (lit("true")) {
            v.kind = Json::BOOL;
            v.b = true;
            return true;
        }
        if (lit("false")) {
            v.kind = Json::BOOL;
            return true;
        }
        if (lit("null")) return true;
        // a number: integers exactly (up to 2^64 - 1), others as double
        const char* q = p;
        if (q < end && (*q == '-' || *q == '+')) ++q;
        bool integral = true;
        while (q < end && ((*q >= '0' && *q <= '9') || *q == '.' || *q == 'e' || *q == 'E' || *q == '-' || *q == '+')) {
            if (*q == '.' || *q == 'e' || *q == 'E') integral = false;
            ++q;
        }
        if (q == p) return false;
        std::string t(p, q);
        v.kind = Json::NUM;
        v.integral = integral && t[0] != '-';
        v.num = strtod(t.c_str(), nullptr);
        if (v.integral) v.u = strtoull(t.c_str(), nullptr, 10);
        p = q;
        return true;
    }
};

static bool parse_json(const char* text, size_t n, Json& out) {
    Parser ps{text, text + n};
    if (!ps.value(out, 0)) return false;
    ps.ws();
    return ps.p == ps.end;
}

// ---- safetensors files (core/safetensors.zig): an 8-byte little-endian header length, the JSON header, the data

enum DType : int { BOOL_, U8, I8, U16, I16, F16, BF16, U32, I32, F32, U64, I64, F64 };
static int dtype_parse(const std::string& t) {
    static const char* names[] = {"BOOL", "U8", "I8", "U16", "I16", "F16", "BF16", "U32", "I32", "F32", "U64", "I64", "F64"};
    for (int i = 0; i < 13; ++i)
        if (t == names[i]) return i;
    return -1;
}
static size_t dtype_size(int d) {
    static const size_t sz[] = {1, 1, 1, 2, 2, 2, 2, 4, 4, 4, 8, 8, 8};
    return d >= 0 && d < 13 ? sz[d] : 0;
}

constexpr int MAX_RANK = 8;

struct Entry {
    int dtype = -1;
    int rank = 0;
    uint64_t shape[MAX_RANK] = {};
    uint64_t begin = 0, end = 0;
};

struct File {
    int fd = -1;
    void* map = nullptr;
    size_t size = 0;
    const uint8_t* data = nullptr;  // the data region (8 + header length)
    std::map<std::string, Entry> entries;
    ~File() {
        if (map && map != MAP_FAILED) munmap(map, size);
        if (fd >= 0) close(fd);
    }
};

static int open_file(const std::string& path, std::unique_ptr<File>& out) {
    auto f = std::make_unique<File>();
    f->fd = open(path.c_str(), O_RDONLY);
    if (f->fd < 0) return EA_BANK_IO;
    struct stat stt;
    if (fstat(f->fd, &stt) != 0) return EA_BANK_IO;
    f->size = (size_t)stt.st_size;
    if (f->size < 8) return EA_BAD_SAFETENSORS;
    f->map = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (f->map == MAP_FAILED) return EA_BANK_IO;
    const uint8_t* b = static_cast<const uint8_t*>(f->map);
    uint64_t hl = 0;
    for (int i = 7; i >= 0; --i) hl = (hl << 8) | b[i];
    if (hl > f->size - 8) return EA_BAD_SAFETENSORS;
    Json h;
    if (!parse_json(reinterpret_cast<const char*>(b + 8), (size_t)hl, h) || h.kind != Json::OBJ) return EA_BAD_SAFETENSORS;
    f->data = b + 8 + hl;
    const size_t data_len = f->size - 8 - (size_t)hl;
    for (const auto& kv : h.obj) {
        if (kv.first == "__metadata__") continue;
        const Json& o = kv.second;
        if (o.kind != Json::OBJ) return EA_BAD_SAFETENSORS;
        const Json* dt = o.get("dtype");
        const Json* sh = o.get("shape");
        const Json* of = o.get("data_offsets");
        if (!dt || dt->kind != Json::STR || !sh || sh->kind != Json::ARR || !of || of->kind != Json::ARR ||
            of->arr.size() != 2)
            return EA_BAD_SAFETENSORS;
        Entry e;
        e.dtype = dtype_parse(dt->s);
        if (e.dtype < 0) return EA_BAD_SAFETENSORS;
        if (sh->arr.size() > MAX_RANK) return EA_BAD_SAFETENSORS;
        e.rank = (int)sh->arr.size();
        uint64_t n = dtype_size(e.dtype);
        for (int i = 0; i < e.rank; ++i) {
            const Json& d = sh->arr[i];
            if (d.kind != Json::NUM || !d.integral) return EA_BAD_SAFETENSORS;
            e.shape[i] = d.u;
            if (__builtin_mul_overflow(n, (uint64_t)d.u, &n)) return EA_BAD_SAFETENSORS;  // no such file fits
        }
        for (int i = 0; i < 2; ++i)
            if (of->arr[i].kind != Json::NUM || !of->arr[i].integral) return EA_BAD_SAFETENSORS;
        e.begin = of->arr[0].u;
        e.end = of->arr[1].u;
        if (e.end < e.begin || e.end - e.begin != n || e.end > data_len) return EA_BAD_SAFETENSORS;
        f->entries[kv.first] = e;
    }
    out = std::move(f);
    return EA_OK;
}

// ---- the split rules of one tensor-parallel rank (split.zig)

enum Rule { REP, ROW, DIM1 };
constexpr uint64_t HAD = 128, TILE = 16;

static bool ends_with(const std::string& s, const std::string& t) {
    return s.size() >= t.size() && s.compare(s.size() - t.size(), t.size(), t) == 0;
}

// The split rules of the tensors this library reads, the MoE block's (split.zig:18-77 holds the whole model's table,
// attention and MTP included, with the same rule for these names). An EXL3 linear of the block -- a routed expert, a
// shared expert, a dense MLP projection -- is cut by its projection's role: gate and up split their outputs (the
// trellis' tile columns and svh), down its inputs (the trellis' tile rows and suh); codebook markers and the scale on
// the uncut side stay whole. The router's weight and score-correction bias stay whole. Any other name has no rule.
static int rule_of(const std::string& name, Rule& r) {
    if (ends_with(name, ".mlp.gate.weight") || ends_with(name, ".mlp.gate.e_score_correction_bias")) {
        r = REP;
        return EA_OK;
    }
    const size_t dot = name.rfind('.');
    if (dot == std::string::npos) return EA_NO_SPLIT_RULE;
    const std::string part = name.substr(dot + 1), stem = name.substr(0, dot);
    const bool in_block = stem.find(".mlp.experts.") != std::string::npos ||
                          stem.find(".mlp.shared_experts.") != std::string::npos ||
                          stem.find(".mlp.gate_proj") != std::string::npos ||
                          stem.find(".mlp.up_proj") != std::string::npos || stem.find(".mlp.down_proj") != std::string::npos;
    if (!in_block) return EA_NO_SPLIT_RULE;
    enum { OUT, IN } role;
    if (ends_with(stem, "gate_proj") || ends_with(stem, "up_proj")) role = OUT;
    else if (ends_with(stem, "down_proj")) role = IN;
    else return EA_NO_SPLIT_RULE;
    if (part == "mcg" || part == "mul1") r = REP;
    else if (part == "trellis") r = role == OUT ? DIM1 : ROW;
    else if (part == "svh") r = role == OUT ? ROW : REP;
    else if (part == "suh") r = role == IN ? ROW : REP;
    else return EA_NO_SPLIT_RULE;
    return EA_OK;
}

// split.zig:61-73: the cut axis divides evenly and no share straddles a Hadamard block.
static int check_cut(const std::string& name, Rule r, const Entry& e, uint64_t world) {
    if (r == REP) return EA_OK;
    const int axis = r == ROW ? 0 : 1;
    if (e.rank <= axis || e.shape[axis] % world != 0) return EA_UNEVEN_SPLIT;
    if (ends_with(name, ".trellis")) {
        if ((e.shape[axis] / world) % (HAD / TILE) != 0) return EA_STRADDLES_HADAMARD;
    } else if (ends_with(name, ".suh") || ends_with(name, ".svh")) {
        if ((e.shape[0] / world) % HAD != 0) return EA_STRADDLES_HADAMARD;
    }
    return EA_OK;
}

struct Share {
    int dtype = -1;
    int rank = 0;
    uint64_t shape[MAX_RANK] = {};
    std::vector<uint8_t> bytes;
};

// weights.zig cut: a whole tensor's share on `rank` of `world`.
static int cut(const File& f, const Entry& e, Rule r, uint64_t rank, uint64_t world, const std::string& name, Share& s) {
    s.dtype = e.dtype;
    s.rank = e.rank;
    std::copy(e.shape, e.shape + MAX_RANK, s.shape);
    const uint8_t* src = f.data + e.begin;
    const uint64_t nbytes = e.end - e.begin;
    if (r == REP) {
        s.bytes.assign(src, src + nbytes);
        return EA_OK;
    }
    int rc = check_cut(name, r, e, world);
    if (rc) return rc;
    if (nbytes == 0) {  // a tensor with a zero dimension: an empty share of the cut shape
        s.shape[r == ROW ? 0 : 1] = e.shape[r == ROW ? 0 : 1] / world;
        s.bytes.clear();
        return EA_OK;
    }
    if (r == ROW) {
        const uint64_t n = e.shape[0] / world, per = nbytes / e.shape[0];
        s.shape[0] = n;
        s.bytes.assign(src + rank * n * per, src + (rank + 1) * n * per);
        return EA_OK;
    }
    const uint64_t n = e.shape[1] / world, inner = nbytes / (e.shape[0] * e.shape[1]);
    s.shape[1] = n;
    s.bytes.resize(e.shape[0] * n * inner);
    for (uint64_t i = 0; i < e.shape[0]; ++i)
        memcpy(s.bytes.data() + i * n * inner, src + (i * e.shape[1] + rank * n) * inner, n * inner);
    return EA_OK;
}

// weights.zig join: the rank's share from its k stored ranks' parts (the same dtype and shape each), in order along
// the cut axis.
static int join(const std::vector<std::pair<const File*, const Entry*>>& parts, Rule r, Share& s) {
    const Entry& p0 = *parts[0].second;
    for (const auto& pe : parts) {
        const Entry& p = *pe.second;
        if (p.dtype != p0.dtype || p.rank != p0.rank || !std::equal(p.shape, p.shape + p.rank, p0.shape))
            return EA_STORED_SHARES_DIFFER;
    }
    s.dtype = p0.dtype;
    s.rank = p0.rank;
    std::copy(p0.shape, p0.shape + MAX_RANK, s.shape);
    const uint64_t pb = p0.end - p0.begin, k = parts.size();
    if (pb == 0 && r != REP) {  // parts with a zero dimension: an empty share of the joined shape
        if (r == DIM1 && p0.rank < 2) return EA_STORED_SHARES_DIFFER;
        s.shape[r == ROW ? 0 : 1] = p0.shape[r == ROW ? 0 : 1] * k;
        s.bytes.clear();
        return EA_OK;
    }
    if (r == REP) {
        const uint8_t* src = parts[0].first->data + p0.begin;
        s.bytes.assign(src, src + pb);
        return EA_OK;
    }
    s.bytes.resize(pb * k);
    if (r == ROW) {
        s.shape[0] = p0.shape[0] * k;
        for (uint64_t i = 0; i < k; ++i)
            memcpy(s.bytes.data() + i * pb, parts[i].first->data + parts[i].second->begin, pb);
        return EA_OK;
    }
    if (p0.rank < 2) return EA_STORED_SHARES_DIFFER;
    const uint64_t rows = p0.shape[0], cols = p0.shape[1], inner = pb / (rows * cols);
    s.shape[1] = cols * k;
    for (uint64_t i = 0; i < rows; ++i)
        for (uint64_t q = 0; q < k; ++q)
            memcpy(s.bytes.data() + (i * cols * k + q * cols) * inner,
                   parts[q].first->data + parts[q].second->begin + i * cols * inner, cols * inner);
    return EA_OK;
}

}  // namespace bank
}  // namespace ea

using namespace ea::bank;

// weights.Reader: a checkpoint directory (or one file of it) read for one rank of `world`; stored_world ranks of
// pre-sharded tensors ("...P_proj.rank{s}.S") are joined k = stored_world / world at a time.
struct ea_bank {
    std::string dir;
    uint64_t rank = 0, world = 1, stored_world = 1;
    std::map<std::string, std::string> index;  // tensor name -> file
    std::map<std::string, std::unique_ptr<File>> files;

    int file(const std::string& fname, File*& out) {
        auto it = files.find(fname);
        if (it != files.end()) {
            out = it->second.get();
            return EA_OK;
        }
        std::unique_ptr<File> f;
        const int rc = open_file(dir + "/" + fname, f);
        if (rc) return rc;
        out = f.get();
        files[fname] = std::move(f);
        return EA_OK;
    }
    int tensor(const std::string& stored, File*& f, const Entry*& e) {
        auto it = index.find(stored);
        if (it == index.end()) return EA_MISSING_TENSOR;
        int rc = file(it->second, f);
        if (rc) return rc;
        auto et = f->entries.find(stored);
        if (et == f->entries.end()) return EA_MISSING_TENSOR;
        e = &et->second;
        return EA_OK;
    }
    static std::string stored_name(const std::string& name, uint64_t s) {
        const size_t dot = name.rfind('.');
        if (dot == std::string::npos) return name;
        return name.substr(0, dot) + ".rank" + std::to_string(s) + name.substr(dot);
    }
    bool has(const std::string& name) const {
        return index.count(name) || index.count(stored_name(name, 0));
    }
    // weights.zig getShare
    int get(const std::string& name, Share& s) {
        Rule r = REP;
        int rc = rule_of(name, r);
        if (index.count(name)) {
            if (rc) return rc;
            File* f;
            const Entry* e;
            if ((rc = tensor(name, f, e))) return rc;
            return cut(*f, *e, r, rank, world, name, s);
        }
        if (rc) return rc;
        const uint64_t k = stored_world / world;
        if (k == 0 || k > 16) return EA_TOO_MANY_STORED_RANKS;
        std::vector<std::pair<const File*, const Entry*>> parts;
        for (uint64_t i = 0; i < k; ++i) {
            File* f;
            const Entry* e;
            if ((rc = tensor(stored_name(name, rank * k + i), f, e))) return rc;
            parts.emplace_back(f, e);
        }
        return join(parts, r, s);
    }
};

namespace {

int bank_check_world(uint32_t rank, uint32_t world, uint32_t stored_world) {
    if (world == 0 || rank >= world || stored_world == 0) return EA_BAD_ARGUMENT;
    if (stored_world % world != 0) return EA_STORED_WORLD_NOT_MULTIPLE;
    return EA_OK;
}

}  // namespace

extern "C" {

static int ea_bank_open_body(const char* dir, uint32_t rank, uint32_t world, uint32_t stored_world, ea_bank** out) {
    if (!dir || !out) return EA_BAD_ARGUMENT;
    int rc = bank_check_world(rank, world, stored_world);
    if (rc) return rc;
    auto b = std::make_unique<ea_bank>();
    b->dir = dir;
    b->rank = rank;
    b->world = world;
    b->stored_world = stored_world;
    const std::string path = b->dir + "/model.safetensors.index.json";
    FILE* fp = fopen(path.c_str(), "rb");
    if (!fp) return EA_BANK_IO;
    std::string text;
    char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof(buf), fp)) > 0) text.append(buf, n);
    fclose(fp);
    Json j;
    if (!parse_json(text.data(), text.size(), j) || j.kind != Json::OBJ) return EA_BAD_INDEX;
    const Json* wm = j.get("weight_map");
    if (!wm || wm->kind != Json::OBJ) return EA_BAD_INDEX;
    for (const auto& kv : wm->obj) {
        if (kv.second.kind != Json::STR) return EA_BAD_INDEX;
        b->index[kv.first] = kv.second.s;
    }
    *out = b.release();
    return EA_OK;
}

static int ea_bank_open_file_body(const char* dir, const char* fname, uint32_t rank, uint32_t world, uint32_t stored_world,
                      ea_bank** out) {
    if (!dir || !fname || !out) return EA_BAD_ARGUMENT;
    int rc = bank_check_world(rank, world, stored_world);
    if (rc) return rc;
    auto b = std::make_unique<ea_bank>();
    b->dir = dir;
    b->rank = rank;
    b->world = world;
    b->stored_world = stored_world;
    File* f;
    if ((rc = b->file(fname, f))) return rc;
    for (const auto& kv : f->entries) b->index[kv.first] = fname;
    *out = b.release();
    return EA_OK;
}

void ea_bank_close(ea_bank* b) { delete b; }

int ea_bank_has(const ea_bank* b, const char* name) {
    try {
        return b && name && b->has(name) ? 1 : 0;
    } catch (...) {  // a failed host allocation: not found
        return 0;
    }
}

static int ea_bank_share_body(ea_bank* b, const char* name, ea_share_info* info, void* dst, uint64_t cap) {
    if (!b || !name || !info) return EA_BAD_ARGUMENT;
    Share s;
    const int rc = b->get(name, s);
    if (rc) return rc;
    info->dtype = s.dtype;
    info->rank = (uint32_t)s.rank;
    for (int i = 0; i < 8; ++i) info->shape[i] = i < s.rank ? s.shape[i] : 1;
    info->bytes = s.bytes.size();
    if (dst) {
        if (cap < s.bytes.size()) return EA_BAD_ARGUMENT;
        memcpy(dst, s.bytes.data(), s.bytes.size());
    }
    return EA_OK;
}

}  // extern "C"

// ---- one layer's routed experts on the device (moe.zig:65-225) ----------------------------------------------------

struct ea_layer {
    ea_routed r{};
    void* slab[3] = {};             // gate, up, down: every expert's trellis back to back, each 256-byte aligned
    void* tables[6] = {};           // ptr[3] (int64 [E]) and k2[3] (int32 [E])
    void* scales[6] = {};           // suh_g, svh_g, suh_u, svh_u, suh_d, svh_d: fp16 [E, K] / [E, N]
    size_t scale_bytes[6] = {};     // one expert's bytes of each
    int device = 0;
    ~ea_layer() {
        (void)hipSetDevice(device);
        for (void* p : slab)
            if (p) (void)hipFree(p);
        for (void* p : tables)
            if (p) (void)hipFree(p);
        for (void* p : scales)
            if (p) (void)hipFree(p);
    }
};

namespace {

const char* PROJ[3] = {"gate", "up", "down"};

std::string xname(uint32_t layer, uint32_t e, int p, const char* part) {
    char buf[192];
    snprintf(buf, sizeof(buf), "model.layers.%u.mlp.experts.%u.%s_proj.%s", layer, e, PROJ[p], part);
    return buf;
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

int hipst(hipError_t e) {
    if (e == hipSuccess) return EA_OK;
    return e == hipErrorOutOfMemory ? EA_OUT_OF_DEVICE_MEMORY : EA_HIP_FAILED;
}

// moe.zig:212-218 codebook: the marker of one expert's projection (1 mcg, 2 mul1, 0 none: 3inst).
uint32_t codebook(const ea_bank* r, uint32_t layer, uint32_t e, int p) {
    if (r->has(xname(layer, e, p, "mcg"))) return 1;
    if (r->has(xname(layer, e, p, "mul1"))) return 2;
    return 0;
}

// One expert's three projections read and checked on the host (trellis i16 [K/16, N/16, 8 K2], fp16 scales).
struct ExpertRead {
    Share tr[3], su[3], sv[3];
};

int read_expert(ea_bank* r, uint32_t layer, uint32_t e, ExpertRead& rd, bool swap) {
    for (int p = 0; p < 3; ++p) {
        int rc;
        if ((rc = r->get(xname(layer, e, p, "trellis"), rd.tr[p]))) return rc;
        if ((rc = r->get(xname(layer, e, p, "suh"), rd.su[p]))) return rc;
        if ((rc = r->get(xname(layer, e, p, "svh"), rd.sv[p]))) return rc;
        const Share& t = rd.tr[p];
        if (t.dtype != I16 || t.rank != 3 || t.shape[2] % 8 != 0) return swap ? EA_SWAP_BAD_TRELLIS : EA_BAD_TRELLIS;
        if (rd.su[p].dtype != F16 || rd.sv[p].dtype != F16) return swap ? EA_SWAP_BAD_SCALES : EA_PACKED_SCALES;
    }
    return EA_OK;
}

}  // namespace

extern "C" {

static int ea_layer_load_body(ea_bank* const* readers, uint32_t nreaders, const uint8_t* pick, uint32_t layer, uint32_t experts,
                  ea_layer** out) {
    if (!readers || nreaders == 0 || !out || experts == 0 || experts > 4096) return EA_BAD_ARGUMENT;
    for (uint32_t i = 0; i < nreaders; ++i)
        if (!readers[i]) return EA_BAD_ARGUMENT;
    if (pick)
        for (uint32_t e = 0; e < experts; ++e)
            if (pick[e] >= nreaders) return EA_BAD_ARGUMENT;
    const uint32_t E = experts;
    auto src = [&](uint32_t e) { return readers[pick ? pick[e] : 0]; };
    std::vector<ExpertRead> rd(E);
    for (uint32_t e = 0; e < E; ++e) {
        const int rc = read_expert(src(e), layer, e, rd[e], false);
        if (rc) return rc;
    }
    const Share& t0 = rd[0].tr[0];
    const uint32_t D = (uint32_t)(t0.shape[0] * 16), I = (uint32_t)(t0.shape[1] * 16);
    for (uint32_t e = 0; e < E; ++e)
        for (int p = 0; p < 3; ++p) {
            const Share& t = rd[e].tr[p];
            const uint64_t K = p == 2 ? I : D, N = p == 2 ? D : I;
            if (t.shape[0] * 16 != K || t.shape[1] * 16 != N) return EA_BAD_TRELLIS;
            if (rd[e].su[p].bytes.size() != K * 2 || rd[e].sv[p].bytes.size() != N * 2) return EA_PACKED_SCALES;
        }
    // moe.zig:143-149: one codebook for the layer, every expert's projections alike when experts come from several banks
    const uint32_t cb = codebook(src(0), layer, 0, 0);
    if (pick)
        for (uint32_t e = 0; e < E; ++e)
            for (int p = 0; p < 3; ++p)
                if (codebook(src(e), layer, e, p) != cb) return EA_MIXED_CODEBOOKS;
    auto L = std::make_unique<ea_layer>();
    int rc = hipst(hipGetDevice(&L->device));
    if (rc) return rc;
    ea_routed& r = L->r;
    r.count = E;
    r.dims = D;
    r.width = I;
    r.cb = cb;
    uint32_t k2lo[3] = {99, 99, 99}, k2hi[3] = {0, 0, 0};
    for (int p = 0; p < 3; ++p) {
        size_t total = 0;
        for (uint32_t e = 0; e < E; ++e) total += align256(rd[e].tr[p].bytes.size());
        if ((rc = hipst(hipMalloc(&L->slab[p], total)))) return rc;
        std::vector<int64_t> ptrs(E);
        std::vector<int32_t> k2(E);
        size_t off = 0;
        for (uint32_t e = 0; e < E; ++e) {
            const Share& t = rd[e].tr[p];
            char* dst = static_cast<char*>(L->slab[p]) + off;
            if ((rc = hipst(hipMemcpy(dst, t.bytes.data(), t.bytes.size(), hipMemcpyHostToDevice)))) return rc;
            ptrs[e] = (int64_t)reinterpret_cast<uintptr_t>(dst);
            k2[e] = (int32_t)(t.shape[2] / 8);
            k2lo[p] = std::min(k2lo[p], (uint32_t)k2[e]);
            k2hi[p] = std::max(k2hi[p], (uint32_t)k2[e]);
            off += align256(t.bytes.size());
        }
        if ((rc = hipst(hipMalloc(&L->tables[p], E * 8)))) return rc;
        if ((rc = hipst(hipMalloc(&L->tables[3 + p], E * 4)))) return rc;
        if ((rc = hipst(hipMemcpy(L->tables[p], ptrs.data(), E * 8, hipMemcpyHostToDevice)))) return rc;
        if ((rc = hipst(hipMemcpy(L->tables[3 + p], k2.data(), E * 4, hipMemcpyHostToDevice)))) return rc;
        r.ptr[p] = reinterpret_cast<uintptr_t>(L->tables[p]);
        r.k2[p] = reinterpret_cast<uintptr_t>(L->tables[3 + p]);
    }
    r.k2_gu[0] = std::min(k2lo[0], k2lo[1]);
    r.k2_gu[1] = std::max(k2hi[0], k2hi[1]);
    r.k2_d[0] = k2lo[2];
    r.k2_d[1] = k2hi[2];
    // stacked scales [E, n] (moe.zig:220-233 stack)
    for (int p = 0; p < 3; ++p)
        for (int j = 0; j < 2; ++j) {
            const int s = 2 * p + j;
            const size_t per = j == 0 ? rd[0].su[p].bytes.size() : rd[0].sv[p].bytes.size();
            L->scale_bytes[s] = per;
            std::vector<uint8_t> host(per * E);
            for (uint32_t e = 0; e < E; ++e) {
                const std::vector<uint8_t>& b = j == 0 ? rd[e].su[p].bytes : rd[e].sv[p].bytes;
                memcpy(host.data() + e * per, b.data(), per);
            }
            if ((rc = hipst(hipMalloc(&L->scales[s], host.size())))) return rc;
            if ((rc = hipst(hipMemcpy(L->scales[s], host.data(), host.size(), hipMemcpyHostToDevice)))) return rc;
        }
    r.suh_g = reinterpret_cast<uintptr_t>(L->scales[0]);
    r.svh_g = reinterpret_cast<uintptr_t>(L->scales[1]);
    r.suh_u = reinterpret_cast<uintptr_t>(L->scales[2]);
    r.svh_u = reinterpret_cast<uintptr_t>(L->scales[3]);
    r.suh_d = reinterpret_cast<uintptr_t>(L->scales[4]);
    r.svh_d = reinterpret_cast<uintptr_t>(L->scales[5]);
    *out = L.release();
    return EA_OK;
}

const ea_routed* ea_layer_routed(const ea_layer* l) { return l ? &l->r : nullptr; }

void ea_layer_free(ea_layer* l) { delete l; }

// expert_swap.zig:345-467 swapLayer, in three steps so that a failure leaves the layer as it was: the changed experts
// read and checked on the host, the three new slabs allocated, then the device written (the slabs: unchanged experts
// copied on the device, changed ones uploaded; their scales overwritten; the ptr / k2 tables rewritten in place, where
// captured graphs hold their addresses) and the old slabs freed. The K2 ranges only widen. Synchronous.
static int ea_layer_swap_body(ea_layer* l, ea_bank* const* banks, uint32_t layer, const uint8_t* target, const uint8_t* current,
                  ea_swap_stats* st) {
    if (!l || !banks || !target || !current) return EA_BAD_ARGUMENT;
    ea_routed& x = l->r;
    const uint32_t E = x.count;
    for (uint32_t j = 0; j < E; ++j) {
        if (target[j] == current[j]) continue;
        // the widths every kernel of this library decodes (K2 4..10), as the reference refuses widths its kernels do
        // not take (expert_swap.zig:94-98: 2..4 bits, 5 with its K10 kernels): a captured graph then always replays
        // on widths its kernels decode
        if (target[j] < 2 || target[j] > 5) return EA_SWAP_WIDTH_UNSUPPORTED;
        if (!banks[target[j]]) return EA_SWAP_NO_BANK;
    }
    int rc = hipst(hipSetDevice(l->device));
    if (rc) return rc;
    // 1. read and check
    std::vector<std::unique_ptr<ExpertRead>> reads(E);
    for (uint32_t j = 0; j < E; ++j) {
        if (target[j] == current[j]) continue;
        ea_bank* r = banks[target[j]];
        uint32_t cb = 99;
        for (int p = 0; p < 3; ++p) {
            const uint32_t c = codebook(r, layer, j, p);
            if (cb != 99 && c != cb) return EA_SWAP_CODEBOOK_DIFFERS;
            cb = c;
        }
        if (cb != x.cb) return EA_SWAP_CODEBOOK_DIFFERS;
        reads[j] = std::make_unique<ExpertRead>();
        if ((rc = read_expert(r, layer, j, *reads[j], true))) return rc;
        const uint64_t k2 = 2ull * target[j];
        for (int p = 0; p < 3; ++p) {
            const Share& t = reads[j]->tr[p];
            const uint64_t K = p == 2 ? x.width : x.dims, N = p == 2 ? x.dims : x.width;
            if (t.shape[0] * 16 != K || t.shape[1] * 16 != N || t.shape[2] != k2 * 8) return EA_SWAP_BAD_TRELLIS;
            if (reads[j]->su[p].bytes.size() != l->scale_bytes[2 * p] ||
                reads[j]->sv[p].bytes.size() != l->scale_bytes[2 * p + 1])
                return EA_SWAP_BAD_SCALES;
        }
    }
    // 2. the new slabs
    const size_t per_k2 = (size_t)x.dims * x.width / 16;  // one expert's trellis bytes a unit of K2 on this rank
    std::vector<int64_t> old_ptrs[3];
    std::vector<int32_t> old_k2[3];
    for (int p = 0; p < 3; ++p) {
        old_ptrs[p].resize(E);
        old_k2[p].resize(E);
        if ((rc = hipst(hipMemcpy(old_ptrs[p].data(), l->tables[p], E * 8, hipMemcpyDeviceToHost)))) return rc;
        if ((rc = hipst(hipMemcpy(old_k2[p].data(), l->tables[3 + p], E * 4, hipMemcpyDeviceToHost)))) return rc;
    }
    void* nb[3] = {};
    for (int p = 0; p < 3; ++p) {
        size_t total = 0;
        for (uint32_t j = 0; j < E; ++j)
            total += align256(reads[j] ? reads[j]->tr[p].bytes.size() : per_k2 * (size_t)old_k2[p][j]);
        if ((rc = hipst(hipMalloc(&nb[p], total)))) {
            for (int q = 0; q < p; ++q) (void)hipFree(nb[q]);
            return rc;
        }
    }
    // 3. the new slabs filled (unchanged experts copied on the device, changed ones uploaded) and the tables built on
    // the host; nothing the layer's kernels read is written yet, so a failure here frees the new slabs and leaves the
    // layer as it was
    auto free_new = [&]() {
        for (void* q : nb) (void)hipFree(q);
    };
    uint64_t read_bytes = 0;
    std::vector<int64_t> ptrs[3];
    std::vector<int32_t> k2v[3];
    uint32_t lo[3] = {99, 99, 99}, hi[3] = {0, 0, 0};
    for (int p = 0; p < 3; ++p) {
        ptrs[p].resize(E);
        k2v[p].resize(E);
        size_t off = 0;
        for (uint32_t j = 0; j < E; ++j) {
            char* dst = static_cast<char*>(nb[p]) + off;
            if (reads[j]) {
                const ExpertRead& rd = *reads[j];
                rc = hipst(hipMemcpy(dst, rd.tr[p].bytes.data(), rd.tr[p].bytes.size(), hipMemcpyHostToDevice));
                k2v[p][j] = (int32_t)(rd.tr[p].shape[2] / 8);
                off += align256(rd.tr[p].bytes.size());
                read_bytes += rd.tr[p].bytes.size() + rd.su[p].bytes.size() + rd.sv[p].bytes.size();
            } else {
                const size_t n = per_k2 * (size_t)old_k2[p][j];
                rc = hipst(hipMemcpy(dst, reinterpret_cast<void*>(static_cast<uintptr_t>(old_ptrs[p][j])), n,
                                     hipMemcpyDeviceToDevice));
                k2v[p][j] = old_k2[p][j];
                off += align256(n);
            }
            if (rc) {
                free_new();
                return rc;
            }
            ptrs[p][j] = (int64_t)reinterpret_cast<uintptr_t>(dst);
            lo[p] = std::min(lo[p], (uint32_t)k2v[p][j]);
            hi[p] = std::max(hi[p], (uint32_t)k2v[p][j]);
        }
    }
    // the changed experts' present scales, kept on the host to put back if a write below fails
    std::vector<std::vector<uint8_t>> old_scales(6);
    for (int s = 0; s < 6; ++s) {
        old_scales[s].resize((size_t)E * l->scale_bytes[s]);
        for (uint32_t j = 0; j < E && !rc; ++j)
            if (reads[j])
                rc = hipst(hipMemcpy(old_scales[s].data() + j * l->scale_bytes[s],
                                     static_cast<char*>(l->scales[s]) + j * l->scale_bytes[s], l->scale_bytes[s],
                                     hipMemcpyDeviceToHost));
        if (rc) {
            free_new();
            return rc;
        }
    }
    // 4. the layer written: the changed experts' scales, then the ptr / k2 tables in place (the graphs hold their
    // addresses). A failed write puts back every scale and table entry written so far before the new slabs go.
    for (uint32_t j = 0; j < E && !rc; ++j) {
        if (!reads[j]) continue;
        for (int p = 0; p < 3 && !rc; ++p) {
            const ExpertRead& rd = *reads[j];
            rc = hipst(hipMemcpy(static_cast<char*>(l->scales[2 * p]) + j * l->scale_bytes[2 * p],
                                 rd.su[p].bytes.data(), rd.su[p].bytes.size(), hipMemcpyHostToDevice));
            if (!rc)
                rc = hipst(hipMemcpy(static_cast<char*>(l->scales[2 * p + 1]) + j * l->scale_bytes[2 * p + 1],
                                     rd.sv[p].bytes.data(), rd.sv[p].bytes.size(), hipMemcpyHostToDevice));
        }
    }
    for (int p = 0; p < 3 && !rc; ++p) {
        rc = hipst(hipMemcpy(l->tables[p], ptrs[p].data(), E * 8, hipMemcpyHostToDevice));
        if (!rc) rc = hipst(hipMemcpy(l->tables[3 + p], k2v[p].data(), E * 4, hipMemcpyHostToDevice));
    }
    if (rc) {
        for (int p = 0; p < 3; ++p) {
            (void)hipMemcpy(l->tables[p], old_ptrs[p].data(), E * 8, hipMemcpyHostToDevice);
            (void)hipMemcpy(l->tables[3 + p], old_k2[p].data(), E * 4, hipMemcpyHostToDevice);
        }
        for (int s = 0; s < 6; ++s)
            for (uint32_t j = 0; j < E; ++j)
                if (reads[j])
                    (void)hipMemcpy(static_cast<char*>(l->scales[s]) + j * l->scale_bytes[s],
                                    old_scales[s].data() + j * l->scale_bytes[s], l->scale_bytes[s],
                                    hipMemcpyHostToDevice);
        (void)hipDeviceSynchronize();
        free_new();
        return rc;
    }
    for (int p = 0; p < 3; ++p) {
        uint32_t* rg = p == 2 ? x.k2_d : x.k2_gu;
        rg[0] = std::min(rg[0], lo[p]);
        rg[1] = std::max(rg[1], hi[p]);
    }
    for (int p = 0; p < 3; ++p) {
        (void)hipFree(l->slab[p]);
        l->slab[p] = nb[p];
    }
    if (st) {
        *st = ea_swap_stats{};
        for (uint32_t j = 0; j < E; ++j)
            if (target[j] != current[j]) {
                st->experts += 1;
                if (target[j] > current[j]) st->up += 1;
                else st->down += 1;
            }
        st->read_bytes = read_bytes;
    }
    return EA_OK;
}

}  // extern "C"

// The entry points above, with every C++ exception turned into a status before it reaches a C caller: a host
// allocation that fails (std::bad_alloc) is EA_OUT_OF_HOST_MEMORY (Zig's error.OutOfMemory), anything else
// EA_BANK_IO. Nothing is half-done on either path that the status does not describe: the bodies build their results
// in local objects and publish them last.
template <class F>
static int guarded(F&& f) {
    try {
        return f();
    } catch (const std::bad_alloc&) {
        return EA_OUT_OF_HOST_MEMORY;
    } catch (...) {
        return EA_BANK_IO;
    }
}

extern "C" {

int ea_bank_open(const char* dir, uint32_t rank, uint32_t world, uint32_t stored_world, ea_bank** out) {
    return guarded([&] { return ea_bank_open_body(dir, rank, world, stored_world, out); });
}

int ea_bank_open_file(const char* dir, const char* fname, uint32_t rank, uint32_t world, uint32_t stored_world,
                      ea_bank** out) {
    return guarded([&] { return ea_bank_open_file_body(dir, fname, rank, world, stored_world, out); });
}

int ea_bank_share(ea_bank* b, const char* name, ea_share_info* info, void* dst, uint64_t cap) {
    return guarded([&] { return ea_bank_share_body(b, name, info, dst, cap); });
}

int ea_layer_load(ea_bank* const* readers, uint32_t nreaders, const uint8_t* pick, uint32_t layer, uint32_t experts,
                  ea_layer** out) {
    return guarded([&] { return ea_layer_load_body(readers, nreaders, pick, layer, experts, out); });
}

int ea_layer_swap(ea_layer* l, ea_bank* const* banks, uint32_t layer, const uint8_t* target, const uint8_t* current,
                  ea_swap_stats* st) {
    return guarded([&] { return ea_layer_swap_body(l, banks, layer, target, current, st); });
}

}  // extern "C"
