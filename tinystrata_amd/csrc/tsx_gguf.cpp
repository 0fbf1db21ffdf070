// tsx_gguf.cpp - GGUF v3 models for the expert kernels: every shard mapped read-only, the header parsed through a
// bounds-checked cursor, and one layer's routed experts repacked into the [gate | up | down] blobs.
//
// Behaviour follows the reference reader (include/strata/artifact/gguf_reader.hpp:233-666); split models use
// llama.cpp's gguf-split file names and split.* keys, as the reference does (include/strata/artifact/gguf_split.hpp:
// 19-23, gguf_reader.hpp:579-607), parsed and checked here by code of this file's own; the repack follows the engine's loader
// (src/qwen35/q36_engine.cu:1144-1168, expert_blob :1196-1201).  The host copies the three strided parts of every
// blob straight from the mapping with hipMemcpy2DAsync, one call per part for a whole run of experts.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <numeric>
#include <regex>
#include <string>
#include <vector>

#include "tsx_common.hpp"
#include "tsx_gguf.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" little-endian
constexpr uint64_t kMaxArray = 1ull << 24;
constexpr size_t kKeptItems = 64;

enum MetaType : uint32_t { U8 = 0, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 };

struct Meta {
    uint32_t type = U32;
    uint64_t u = 0;  // integers (signed ones sign-extended), bools
    double f = 0;    // F32 / F64
    std::string s;
    uint32_t elem = U32;
    uint64_t count = 0;
    std::vector<Meta> items;  // the first kKeptItems of an array
};

struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t offset = 0;
    uint64_t bytes = 0;
};

struct Fault {
    std::string msg;
};

// a read cursor over the mapped header: every read checks the bytes remaining
class Cursor {
public:
    Cursor(const uint8_t* p, uint64_t n, const std::string& path) : p_(p), n_(n), path_(path) {}
    void need(uint64_t k) const {
        if (k > n_ - pos_) throw Fault{path_ + ": unexpected end of file in the GGUF header"};
    }
    template <typename T> T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p_ + pos_, sizeof(T));
        pos_ += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t k = get<uint64_t>();
        need(k);
        std::string s((const char*) p_ + pos_, (size_t) k);
        pos_ += k;
        return s;
    }
    uint64_t pos() const { return pos_; }

private:
    const uint8_t* p_;
    uint64_t n_, pos_ = 0;
    const std::string& path_;
};

Meta read_meta(Cursor& c, uint32_t type, int depth, const std::string& path) {
    if (depth > 2) throw Fault{path + ": GGUF metadata arrays nested too deep"};
    Meta m;
    m.type = type;
    switch (type) {
        case U8: m.u = c.get<uint8_t>(); break;
        case I8: m.u = (uint64_t) (int64_t) c.get<int8_t>(); break;
        case U16: m.u = c.get<uint16_t>(); break;
        case I16: m.u = (uint64_t) (int64_t) c.get<int16_t>(); break;
        case U32: m.u = c.get<uint32_t>(); break;
        case I32: m.u = (uint64_t) (int64_t) c.get<int32_t>(); break;
        case F32: m.f = c.get<float>(); break;
        case BOOL: m.u = c.get<uint8_t>() != 0; break;
        case STRING: m.s = c.str(); break;
        case U64: m.u = c.get<uint64_t>(); break;
        case I64: m.u = (uint64_t) c.get<int64_t>(); break;
        case F64: m.f = c.get<double>(); break;
        case ARRAY: {
            m.elem = c.get<uint32_t>();
            m.count = c.get<uint64_t>();
            if (m.count > kMaxArray) throw Fault{path + ": implausible GGUF metadata array length"};
            for (uint64_t i = 0; i < m.count; ++i) {
                Meta e = read_meta(c, m.elem, depth + 1, path);
                if (m.items.size() < kKeptItems) m.items.push_back(std::move(e));
            }
            break;
        }
        default: throw Fault{path + ": unknown GGUF metadata value type " + std::to_string(type)};
    }
    return m;
}

bool geometry(uint32_t t, int& elems, int& bytes) {
    // (values, bytes) per block of the ggml type ids a GGUF model carries
    struct G {
        uint32_t id;
        int e, b;
    };
    static const G table[] = {
        {0, 1, 4},      {1, 1, 2},       {2, 32, 18},    {3, 32, 20},     {6, 32, 22},    {7, 32, 24},
        {8, 32, 34},    {9, 32, 36},     {10, 256, 84},  {11, 256, 110},  {12, 256, 144}, {13, 256, 176},
        {14, 256, 210}, {16, 256, 66},   {17, 256, 74},  {18, 256, 98},   {20, 32, 18},   {21, 256, 110},
        {22, 256, 82},  {23, 256, 136},  {24, 1, 1},     {29, 256, 56},   {30, 1, 2},     {39, 32, 17},
        {40, 64, 36},   {42, 64, 18},
    };
    for (const G& g : table)
        if (g.id == t) {
            elems = g.e;
            bytes = g.b;
            return true;
        }
    return false;
}

// payload bytes from the shape and the block geometry; 0 when the type is unknown, a row is not whole blocks or
// the count overflows
uint64_t payload_bytes(const Tensor& t) {
    int be = 0, bb = 0;
    if (t.n_dims == 0 || !geometry(t.type, be, bb) || t.ne[0] % be != 0) return 0;
    uint64_t n = 1;
    for (uint32_t d = 0; d < t.n_dims; ++d) {
        const uint64_t k = (uint64_t) t.ne[d];
        if (k == 0 || n > std::numeric_limits<uint64_t>::max() / k) return 0;
        n *= k;
    }
    const uint64_t blocks = n / (uint64_t) be;
    if (blocks > std::numeric_limits<uint64_t>::max() / (uint64_t) bb) return 0;
    return blocks * (uint64_t) bb;
}

struct Shard {
    std::string path;
    int fd = -1;
    const uint8_t* base = nullptr;
    uint64_t size = 0, data_start = 0, alignment = 32;
    uint32_t version = 0;
    std::vector<Tensor> tensors;
    std::map<std::string, Meta> meta;
    std::vector<std::string> keys;  // metadata keys in file order

    ~Shard() {
        if (base) munmap((void*) base, size);
        if (fd >= 0) ::close(fd);
    }
    const Meta* get(const std::string& k) const {
        const auto it = meta.find(k);
        return it == meta.end() ? nullptr : &it->second;
    }
    // the tensor's payload [data_start + offset, + bytes) ends within the mapping, with no wrap of the sum
    bool inside(const Tensor& t) const {
        uint64_t at = 0, end = 0;
        if (t.bytes == 0 || __builtin_add_overflow(data_start, t.offset, &at)) return false;
        return !__builtin_add_overflow(at, t.bytes, &end) && end <= size;
    }

    void open_map() {
        fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) throw Fault{path + ": cannot open (" + std::strerror(errno) + ")"};
        struct stat st {};
        if (fstat(fd, &st) != 0) throw Fault{path + ": cannot stat"};
        size = (uint64_t) st.st_size;
        if (size == 0) throw Fault{path + ": empty file, not a GGUF model"};
        void* p = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) throw Fault{path + ": mmap failed (" + std::strerror(errno) + ")"};
        base = (const uint8_t*) p;
    }
    void parse() {
        Cursor c(base, size, path);
        if (c.get<uint32_t>() != kMagic) throw Fault{path + ": not a GGUF file (bad magic)"};
        version = c.get<uint32_t>();
        if (version != 3) throw Fault{path + ": GGUF v" + std::to_string(version) + ", this reader handles v3"};
        const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
        for (uint64_t i = 0; i < n_kv; ++i) {
            std::string key = c.str();
            const uint32_t type = c.get<uint32_t>();
            Meta m = read_meta(c, type, 0, path);
            if (meta.emplace(key, std::move(m)).second) keys.push_back(std::move(key));
        }
        std::map<std::string, size_t> seen;
        for (uint64_t i = 0; i < n_tensors; ++i) {
            Tensor t;
            t.name = c.str();
            if (!seen.emplace(t.name, i).second) throw Fault{path + ": duplicate tensor name '" + t.name + "'"};
            t.n_dims = c.get<uint32_t>();
            if (t.n_dims == 0 || t.n_dims > 4) throw Fault{path + ": bad n_dims for " + t.name};
            for (uint32_t d = 0; d < t.n_dims; ++d) {
                const uint64_t k = c.get<uint64_t>();
                if (k > (uint64_t) std::numeric_limits<int64_t>::max())
                    throw Fault{path + ": dimension out of range for " + t.name};
                t.ne[d] = (int64_t) k;
            }
            t.type = c.get<uint32_t>();
            t.offset = c.get<uint64_t>();
            t.bytes = payload_bytes(t);
            tensors.push_back(std::move(t));
        }
        if (const Meta* a = get("general.alignment"))
            if (a->u) alignment = a->u;
        const uint64_t end = c.pos();
        data_start = end + (alignment - end % alignment) % alignment;
        if (data_start > size) {
            // a shard with no tensors (a split model's metadata shard) may end before the aligned data start
            if (n_tensors != 0) throw Fault{path + ": GGUF data section starts past the end of the file"};
            data_start = size;
        }
    }
};

// A split model's file names, as llama.cpp's gguf-split writes them: "<stem>-<index>-of-<count>.gguf" with both
// numbers five digits wide, index 1-based.  parse_split_name takes one such name apart; names of every other form
// belong to models of one file.
struct SplitName {
    std::string stem;  // everything before "-<index>-of-"
    int index = 0, count = 0;
    std::string name(int i) const {
        char digits[32];
        std::snprintf(digits, sizeof digits, "-%05d-of-%05d.gguf", i, count);
        return stem + digits;
    }
};
bool parse_split_name(const std::string& path, SplitName& out) {
    // the file name itself must have a stem: "dir/-00001-of-00002.gguf" is a one-file model
    static const std::regex form(R"(^([^/]+)-([0-9]{5})-of-([0-9]{5})\.gguf$)");
    const size_t slash = path.find_last_of('/');
    const std::string dir = slash == std::string::npos ? std::string() : path.substr(0, slash + 1);
    const std::string file = slash == std::string::npos ? path : path.substr(slash + 1);
    std::smatch m;
    if (!std::regex_match(file, m, form)) return false;
    out.stem = dir + m[1].str();
    out.index = std::stoi(m[2].str());
    out.count = std::stoi(m[3].str());
    return out.count >= 1 && out.index >= 1 && out.index <= out.count;
}
bool readable_file(const std::string& p) {
    struct stat st {};
    return ::stat(p.c_str(), &st) == 0 && S_ISREG(st.st_mode) && ::access(p.c_str(), R_OK) == 0;
}
// every shard of the model `any` belongs to, first shard first; `any` alone when its name is not a split name
std::vector<std::string> split_paths(const std::string& any) {
    SplitName sn;
    if (!parse_split_name(any, sn)) return {any};
    std::vector<std::string> out;
    std::string absent;
    int n_absent = 0;
    for (int i = 1; i <= sn.count; ++i) {
        out.push_back(sn.name(i));
        if (!readable_file(out.back()) && n_absent++ == 0) absent = out.back();
    }
    if (n_absent)
        throw Fault{"split model " + sn.stem + ": " + std::to_string(n_absent) + " of its " + std::to_string(sn.count) +
                    " shard files not found, first " + absent};
    return out;
}

uint64_t lcm64(uint64_t a, uint64_t b) { return a / std::gcd(a, b) * b; }

int fail(int code, const std::string& msg) {
    tsx::set_error("%s", msg.c_str());
    return code;
}

}  // namespace

struct tsx_gguf {
    std::vector<std::unique_ptr<Shard>> shards;
    std::vector<std::pair<int, size_t>> order;         // directory order: (shard, tensor)
    std::map<std::string, std::pair<int, size_t>> by;  // name -> (shard, tensor)

    // The split.* keys must describe exactly the shard set that was opened: every shard says "n shards, I am number
    // i" (split.no counts from 0), all of them quote one tensor total (split.tensors.count, optional) and their
    // directories add up to it, and the model metadata sits in the first shard.  A lone file may not claim to be
    // part of a larger set.
    void check_split() const {
        constexpr uint64_t kNone = ~0ull;
        auto declared = [](const Shard& s, const char* key) {
            const Meta* m = s.get(key);
            return m ? m->u : kNone;
        };
        auto show = [](uint64_t v) { return v == kNone ? std::string("absent") : std::to_string(v); };
        const uint64_t n = shards.size();
        if (n == 1) {
            const uint64_t claim = declared(*shards[0], "split.count");
            if (claim != kNone && claim > 1)
                throw Fault{shards[0]->path + ": split.count is " + std::to_string(claim) +
                            ", so this file alone is not a whole model (open it by its path to find the other shards)"};
            return;
        }
        const uint64_t total = declared(*shards[0], "split.tensors.count");
        uint64_t listed = 0;
        for (uint64_t i = 0; i < n; ++i) {
            const Shard& s = *shards[i];
            std::string bad;
            if (declared(s, "split.count") != n)
                bad = "split.count " + show(declared(s, "split.count")) + ", expected " + std::to_string(n);
            else if (declared(s, "split.no") != i)
                bad = "split.no " + show(declared(s, "split.no")) + ", expected " + std::to_string(i);
            else if (declared(s, "split.tensors.count") != total)
                bad = "split.tensors.count " + show(declared(s, "split.tensors.count")) + " where the first shard has " +
                      show(total);
            if (!bad.empty())
                throw Fault{"shard " + std::to_string(i + 1) + " of " + std::to_string(n) + " (" + s.path +
                            ") does not match the set: " + bad};
            listed += s.tensors.size();
        }
        if (total != kNone && listed != total)
            throw Fault{"split model: split.tensors.count is " + std::to_string(total) + " but the " +
                        std::to_string(n) + " shard directories list " + std::to_string(listed) + " tensors"};
        if (!shards[0]->get("general.architecture"))
            throw Fault{shards[0]->path + ": first shard of a split model without general.architecture (the model "
                                          "metadata belongs there)"};
    }
    void fill(int shard, size_t i, tsx_gguf_tensor* out) const {
        const Shard& s = *shards[shard];
        const Tensor& t = s.tensors[i];
        out->name = t.name.c_str();
        out->type = (int32_t) t.type;
        out->n_dims = (int32_t) t.n_dims;
        for (int d = 0; d < 4; ++d) out->ne[d] = t.ne[d];
        out->offset = t.offset;
        out->bytes = t.bytes;
        out->data = s.inside(t) ? s.base + s.data_start + t.offset : nullptr;
        out->shard = shard;
    }
    const Meta* meta(const char* key) const { return key ? shards[0]->get(key) : nullptr; }
};

extern "C" {

TSX_API int tsx_gguf_block_geometry(int type, int* elems, int* bytes) {
    TSX_REQUIRE(elems && bytes, "tsx_gguf_block_geometry: null output");
    if (type < 0 || !geometry((uint32_t) type, *elems, *bytes))
        return fail(TSX_ERR_UNSUPPORTED, "ggml type " + std::to_string(type) + " has no known block geometry");
    return TSX_OK;
}

TSX_API int tsx_gguf_split_paths(const char* any_shard, char* buf, size_t cap, int* n_paths, size_t* n_bytes) {
    TSX_REQUIRE(any_shard && n_paths && n_bytes, "tsx_gguf_split_paths: null argument");
    try {
        const std::vector<std::string> p = split_paths(any_shard);
        size_t need = 0;
        for (const auto& s : p) need += s.size() + 1;
        *n_paths = (int) p.size();
        *n_bytes = need;
        if (buf == nullptr || cap < need) return fail(TSX_ERR_ARG, "tsx_gguf_split_paths: buffer too small");
        for (const auto& s : p) {
            std::memcpy(buf, s.c_str(), s.size() + 1);
            buf += s.size() + 1;
        }
        return TSX_OK;
    } catch (const Fault& f) {
        return fail(TSX_ERR_NOT_FOUND, f.msg);
    }
}

TSX_API int tsx_gguf_open(const char* const* paths, int n_paths, tsx_gguf** out) {
    TSX_REQUIRE(paths && n_paths > 0 && out, "tsx_gguf_open: paths, n_paths > 0, out");
    *out = nullptr;
    auto g = std::make_unique<tsx_gguf>();
    try {
        for (int i = 0; i < n_paths; ++i) {
            TSX_REQUIRE(paths[i], "tsx_gguf_open: null path %d", i);
            auto s = std::make_unique<Shard>();
            s->path = paths[i];
            s->open_map();
            s->parse();
            g->shards.push_back(std::move(s));
        }
        g->check_split();
        for (int i = 0; i < (int) g->shards.size(); ++i)
            for (size_t t = 0; t < g->shards[i]->tensors.size(); ++t) {
                const std::string& name = g->shards[i]->tensors[t].name;
                const auto ins = g->by.emplace(name, std::make_pair(i, t));
                if (!ins.second)
                    throw Fault{"tensor " + name + " is in two shards (" + g->shards[ins.first->second.first]->path +
                                " and " + g->shards[i]->path + ")"};
                g->order.emplace_back(i, t);
            }
    } catch (const Fault& f) {
        return fail(TSX_ERR_FORMAT, f.msg);
    } catch (const std::bad_alloc&) {
        return fail(TSX_ERR_FORMAT, "tsx_gguf_open: out of host memory while parsing");
    }
    *out = g.release();
    return TSX_OK;
}

TSX_API int tsx_gguf_open_model(const char* any_shard, tsx_gguf** out) {
    TSX_REQUIRE(any_shard && out, "tsx_gguf_open_model: path, out");
    std::vector<std::string> p;
    try {
        p = split_paths(any_shard);
    } catch (const Fault& f) {
        return fail(TSX_ERR_NOT_FOUND, f.msg);
    }
    std::vector<const char*> c;
    for (const auto& s : p) c.push_back(s.c_str());
    return tsx_gguf_open(c.data(), (int) c.size(), out);
}

TSX_API void tsx_gguf_close(tsx_gguf* g) { delete g; }

TSX_API int tsx_gguf_shard_count(const tsx_gguf* g) { return g ? (int) g->shards.size() : 0; }

TSX_API int tsx_gguf_shard_info(const tsx_gguf* g, int shard, uint32_t* version, uint64_t* alignment,
                                uint64_t* data_start, uint64_t* file_size) {
    TSX_REQUIRE(g && shard >= 0 && shard < (int) g->shards.size(), "tsx_gguf_shard_info: no shard %d", shard);
    const Shard& s = *g->shards[shard];
    if (version) *version = s.version;
    if (alignment) *alignment = s.alignment;
    if (data_start) *data_start = s.data_start;
    if (file_size) *file_size = s.size;
    return TSX_OK;
}

TSX_API int64_t tsx_gguf_tensor_count(const tsx_gguf* g) { return g ? (int64_t) g->order.size() : 0; }

TSX_API int tsx_gguf_tensor_at(const tsx_gguf* g, int64_t i, tsx_gguf_tensor* out) {
    TSX_REQUIRE(g && out && i >= 0 && i < (int64_t) g->order.size(), "tsx_gguf_tensor_at: no tensor %lld",
                (long long) i);
    g->fill(g->order[(size_t) i].first, g->order[(size_t) i].second, out);
    return TSX_OK;
}

TSX_API int tsx_gguf_find(const tsx_gguf* g, const char* name, tsx_gguf_tensor* out) {
    TSX_REQUIRE(g && name && out, "tsx_gguf_find: model, name, out");
    const auto it = g->by.find(name);
    if (it == g->by.end()) return fail(TSX_ERR_NOT_FOUND, std::string("no tensor ") + name);
    g->fill(it->second.first, it->second.second, out);
    return TSX_OK;
}

TSX_API int tsx_gguf_meta_count(const tsx_gguf* g) { return g ? (int) g->shards[0]->keys.size() : 0; }

TSX_API const char* tsx_gguf_meta_key(const tsx_gguf* g, int i) {
    if (!g || i < 0 || i >= (int) g->shards[0]->keys.size()) return nullptr;
    return g->shards[0]->keys[(size_t) i].c_str();
}

TSX_API int tsx_gguf_meta(const tsx_gguf* g, const char* key, int* type, uint64_t* u, int64_t* i, double* f,
                          const char** s, int* elem_type, uint64_t* count) {
    TSX_REQUIRE(g && key, "tsx_gguf_meta: model, key");
    const Meta* m = g->meta(key);
    if (!m) return fail(TSX_ERR_NOT_FOUND, std::string("no metadata key ") + key);
    if (type) *type = (int) m->type;
    if (u) *u = m->u;
    if (i) *i = (int64_t) m->u;
    if (f) *f = (m->type == F32 || m->type == F64) ? m->f : (m->type == I8 || m->type == I16 || m->type == I32 ||
                                                             m->type == I64)
                                                                ? (double) (int64_t) m->u
                                                                : (double) m->u;
    if (s) *s = m->type == STRING ? m->s.c_str() : nullptr;
    if (elem_type) *elem_type = m->type == ARRAY ? (int) m->elem : -1;
    if (count) *count = m->type == ARRAY ? m->count : 1;
    return TSX_OK;
}

TSX_API int tsx_gguf_meta_item(const tsx_gguf* g, const char* key, uint64_t item, uint64_t* u, double* f,
                               const char** s) {
    TSX_REQUIRE(g && key, "tsx_gguf_meta_item: model, key");
    const Meta* m = g->meta(key);
    if (!m) return fail(TSX_ERR_NOT_FOUND, std::string("no metadata key ") + key);
    if (m->type != ARRAY || item >= m->items.size())
        return fail(TSX_ERR_NOT_FOUND, std::string(key) + ": no kept array item " + std::to_string(item));
    const Meta& e = m->items[(size_t) item];
    if (u) *u = e.u;
    if (f) *f = (e.type == F32 || e.type == F64) ? e.f : (double) e.u;
    if (s) *s = e.type == STRING ? e.s.c_str() : nullptr;
    return TSX_OK;
}

TSX_API int tsx_gguf_layer_experts(const tsx_gguf* g, int layer, int shared, tsx_gguf_experts* out) {
    TSX_REQUIRE(g && out && layer >= 0, "tsx_gguf_layer_experts: model, layer >= 0, out");
    const std::string pre = "blk." + std::to_string(layer) + ".ffn_";
    const char* sfx = shared ? "_shexp.weight" : "_exps.weight";
    const uint32_t nd = shared ? 2 : 3;
    tsx_gguf_tensor t[3];
    const char* part[3] = {"gate", "up", "down"};
    for (int i = 0; i < 3; ++i) {
        const int rc = tsx_gguf_find(g, (pre + part[i] + sfx).c_str(), &t[i]);
        if (rc != TSX_OK) return rc;
    }
    const tsx_gguf_tensor &tg = t[0], &tu = t[1], &td = t[2];
    const std::string what = pre + "{gate,up,down}" + sfx;
    if (tg.type != tu.type || tg.n_dims != (int) nd || tu.n_dims != (int) nd || td.n_dims != (int) nd ||
        tg.ne[0] != tu.ne[0] || tg.ne[1] != tu.ne[1] || tg.ne[2] != tu.ne[2])
        return fail(TSX_ERR_FORMAT, what + ": gate and up differ in type or shape, or are not [n_embd, n_ff" +
                                        (shared ? "]" : ", n_expert]"));
    const int64_t n_embd = tg.ne[0], n_ff = tg.ne[1], n_exp = tg.ne[2];
    if (td.ne[0] != n_ff || td.ne[1] != n_embd || td.ne[2] != n_exp)
        return fail(TSX_ERR_FORMAT, what + ": down is not [n_ff, n_embd" + (shared ? "]" : ", n_expert]") +
                                        " of the gate's shape");
    if (!tsx_moe_expert_supported(tg.type, td.type, n_embd, n_ff))
        return fail(TSX_ERR_UNSUPPORTED, what + ": types " + std::to_string(tg.type) + "/" + std::to_string(td.type) +
                                             " at " + std::to_string(n_embd) + " x " + std::to_string(n_ff) +
                                             ", which the expert kernels do not take");
    for (int i = 0; i < 3; ++i)
        if (t[i].data == nullptr) return fail(TSX_ERR_FORMAT, std::string(t[i].name) + ": payload outside its file");
    out->L = tsx_make_layout(tg.type, td.type, n_embd, n_ff);
    const uint64_t al = lcm64(lcm64(tsx_type_block_bytes(tg.type), tsx_type_block_bytes(td.type)), 16);
    out->stride = (out->L.bytes + al - 1) / al * al;
    out->n_expert = n_exp;
    out->gate = tg.data;
    out->up = tu.data;
    out->down = td.data;
    return TSX_OK;
}

TSX_API int tsx_gguf_expert_blob(const tsx_gguf_experts* X, int64_t e, void* dst) {
    TSX_REQUIRE(X && dst && e >= 0 && e < X->n_expert, "tsx_gguf_expert_blob: experts, dst, 0 <= e < n_expert");
    const uint64_t gsz = X->L.up_off, dsz = X->L.bytes - X->L.down_off;
    uint8_t* d = (uint8_t*) dst;
    std::memcpy(d, (const uint8_t*) X->gate + (uint64_t) e * gsz, gsz);
    std::memcpy(d + X->L.up_off, (const uint8_t*) X->up + (uint64_t) e * gsz, gsz);
    std::memcpy(d + X->L.down_off, (const uint8_t*) X->down + (uint64_t) e * dsz, dsz);
    return TSX_OK;
}

TSX_API int tsx_gguf_upload_experts(const tsx_gguf_experts* X, int64_t e0, int64_t n, void* dst, uint64_t dst_stride,
                                    void* stream) {
    TSX_REQUIRE(X && dst && e0 >= 0 && n >= 0 && e0 + n <= X->n_expert && dst_stride >= X->L.bytes &&
                    dst_stride % 16 == 0 && tsx::aligned(dst, 16),
                "tsx_gguf_upload_experts: experts, dst (16-byte aligned), 0 <= e0, e0 + n <= n_expert, dst_stride "
                ">= the blob and a multiple of 16");
    if (n == 0) return TSX_OK;
    const uint64_t gsz = X->L.up_off, dsz = X->L.bytes - X->L.down_off;
    const hipStream_t s = (hipStream_t) stream;
    uint8_t* d = (uint8_t*) dst;
    const struct {
        uint64_t off, size;
        const void* src;
    } parts[3] = {{0, gsz, X->gate}, {X->L.up_off, gsz, X->up}, {X->L.down_off, dsz, X->down}};
    for (const auto& p : parts) {
        const hipError_t e = hipMemcpy2DAsync(d + p.off, dst_stride, (const uint8_t*) p.src + (uint64_t) e0 * p.size,
                                              p.size, p.size, (size_t) n, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) {
            tsx::set_error("tsx_gguf_upload_experts: %s", hipGetErrorString(e));
            return (int) e;
        }
    }
    return TSX_OK;
}

}  // extern "C"
