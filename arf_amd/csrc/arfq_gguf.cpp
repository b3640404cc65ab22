// arfq_gguf.cpp -- GGUF v3 reader feeding arfq_weight_upload (host C++).
//
// Follows LazyGguf::open_raw (crates/arf-core/src/model/gguf.rs:509-564): magic,
// version 3, tensor and key/value counts, the key/value section (only
// general.alignment is kept, every other value skipped as Reader::skip_value,
// gguf.rs:323-360), the tensor table (name, dims fastest-varying first, ggml
// type id, offset) and the data section at the header end rounded up to the
// alignment.  The file is memory-mapped; tensor bytes are read in place.
//
// Raw block access follows get_q4k_blocks_raw / get_q8_0_blocks_raw
// (gguf.rs:774-828): a tensor of the requested type, rows = elements / ne0,
// cols = ne0, ggml_byte_len bytes from data_start + offset.  A 3-D `*_exps`
// tensor [ne0, ne1, ne2] uploads as ne2 experts of [ne1 rows, ne0 cols], each
// a whole number of blocks (index_experts, gguf.rs:1479-1523); a row range of
// a 2-D tensor uploads as its own matrix (Entry::RowSlice, gguf.rs:125-140).
//
// Differences from the reference, all on malformed input: general.alignment
// must be a nonzero u32 (the reference reads four bytes whatever the type and
// divides by the value); arrays nest at most 64 deep (the reference recurses
// without a bound); a tensor's bytes are checked against the file size when
// they are read (the reference's slice would panic).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <exception>
#include <new>
#include <string>
#include <vector>

#include "../../include/arfq.h"

struct arfq_gguf_tensor {
    std::string name;
    std::vector<uint64_t> dims;
    int type = 0;
    uint64_t offset = 0;  // relative to the data section
    uint64_t elems = 0;
    uint64_t nbytes = 0;  // ggml_byte_len(type, elems)
};

struct arfq_gguf {
    const uint8_t *map = nullptr;
    size_t size = 0;
    uint64_t alignment = 32;
    uint64_t data_start = 0;
    std::vector<arfq_gguf_tensor> tensors;
    std::string err;
};

namespace {

thread_local std::string g_gguf_err;

// ggml block geometry (gguf.rs:1657-1705): elements per block and bytes per
// block; F32/F16/BF16 count one element as a block.  0 = unsupported type
// (GgmlType::from_id, gguf.rs:60-90).
struct TypeGeom {
    int qk, bytes;
};
TypeGeom type_geom(int t) {
    switch (t) {
    case 0: return {1, 4};      // F32
    case 1: return {1, 2};      // F16
    case 30: return {1, 2};     // BF16
    case 2: return {32, 18};    // Q4_0
    case 3: return {32, 20};    // Q4_1
    case 8: return {32, 34};    // Q8_0
    case 20: return {32, 18};   // IQ4_NL
    case 12: return {256, 144}; // Q4_K
    case 13: return {256, 176}; // Q5_K
    case 14: return {256, 210}; // Q6_K
    case 11: return {256, 110}; // Q3_K
    case 21: return {256, 110}; // IQ3_S
    case 23: return {256, 136}; // IQ4_XS
    default: return {0, 0};
    }
}

struct Reader {
    const uint8_t *buf;
    size_t size, pos = 0;
    bool take(size_t n, const uint8_t **p) {
        if (n > size - pos) return false;
        *p = buf + pos;
        pos += n;
        return true;
    }
    bool u32(uint32_t *v) {
        const uint8_t *p;
        if (!take(4, &p)) return false;
        std::memcpy(v, p, 4);  // little-endian host (x86_64)
        return true;
    }
    bool u64(uint64_t *v) {
        const uint8_t *p;
        if (!take(8, &p)) return false;
        std::memcpy(v, p, 8);
        return true;
    }
    bool string(std::string *s) {
        uint64_t n;
        const uint8_t *p;
        if (!u64(&n) || n > size - pos || !take((size_t)n, &p)) return false;
        s->assign(reinterpret_cast<const char *>(p), (size_t)n);
        return true;
    }
};

// Skip one value of GGUF value type vty (Reader::skip_value, gguf.rs:323-360).
// Returns "" or an error message.
std::string skip_value(Reader &r, uint32_t vty, int depth) {
    const uint8_t *p;
    size_t fixed = 0;
    switch (vty) {
    case 0: case 1: case 7: fixed = 1; break;   // u8 / i8 / bool
    case 2: case 3: fixed = 2; break;           // u16 / i16
    case 4: case 5: case 6: fixed = 4; break;   // u32 / i32 / f32
    case 10: case 11: case 12: fixed = 8; break; // u64 / i64 / f64
    case 8: {                                   // string
        std::string s;
        return r.string(&s) ? "" : "GGUF truncated";
    }
    case 9: {  // array: element type, count, elements
        if (depth >= 64) return "GGUF arrays nested too deep";
        uint32_t ety;
        uint64_t n;
        if (!r.u32(&ety) || !r.u64(&n)) return "GGUF truncated";
        size_t esz = 0;
        switch (ety) {
        case 0: case 1: case 7: esz = 1; break;
        case 2: case 3: esz = 2; break;
        case 4: case 5: case 6: esz = 4; break;
        case 10: case 11: case 12: esz = 8; break;
        default: break;
        }
        if (esz) {  // fixed-size elements: one bounds check for the whole array
            if (n > (r.size - r.pos) / esz) return "GGUF truncated";
            r.pos += (size_t)(n * esz);
            return "";
        }
        for (uint64_t i = 0; i < n; i++) {  // (an unknown element type fails on the first element)
            std::string e = skip_value(r, ety, depth + 1);
            if (!e.empty()) return e;
        }
        return "";
    }
    default:
        return "unknown GGUF value type " + std::to_string(vty);
    }
    return r.take(fixed, &p) ? "" : "GGUF truncated";
}

std::string parse(arfq_gguf *g) {
    Reader r{g->map, g->size};
    const uint8_t *magic;
    if (!r.take(4, &magic) || std::memcmp(magic, "GGUF", 4) != 0) return "not a GGUF file (bad magic)";
    uint32_t version;
    if (!r.u32(&version)) return "GGUF truncated";
    if (version != 3) return "GGUF version " + std::to_string(version) + " unsupported (only v3)";
    uint64_t n_tensors, n_kv;
    if (!r.u64(&n_tensors) || !r.u64(&n_kv)) return "GGUF truncated";
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key;
        uint32_t vty;
        if (!r.string(&key) || !r.u32(&vty)) return "GGUF truncated";
        if (key == "general.alignment") {
            uint32_t a;
            if (vty != 4) return "GGUF general.alignment has value type " + std::to_string(vty) + ", expected u32";
            if (!r.u32(&a)) return "GGUF truncated";
            if (a == 0) return "GGUF general.alignment is 0";
            g->alignment = a;
        } else {
            std::string e = skip_value(r, vty, 0);
            if (!e.empty()) return e;
        }
    }
    // each tensor entry takes at least 24 bytes: bound the count before reserving
    if (n_tensors > (r.size - r.pos) / 24) return "GGUF truncated";
    g->tensors.reserve((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        arfq_gguf_tensor t;
        uint32_t n_dims, ty;
        if (!r.string(&t.name) || !r.u32(&n_dims)) return "GGUF truncated";
        if (n_dims > (r.size - r.pos) / 8) return "GGUF truncated";
        t.dims.resize(n_dims);
        uint64_t elems = 1;
        for (uint32_t d = 0; d < n_dims; d++) {
            if (!r.u64(&t.dims[d])) return "GGUF truncated";
            if (t.dims[d] && elems > UINT64_MAX / t.dims[d]) return "GGUF tensor " + t.name + ": element count overflows";
            elems *= t.dims[d];
        }
        if (!r.u32(&ty) || !r.u64(&t.offset)) return "GGUF truncated";
        const TypeGeom tg = type_geom((int)ty);
        if (!tg.qk) return "unsupported ggml tensor type " + std::to_string(ty) + " (tensor " + t.name + ")";
        t.type = (int)ty;
        t.elems = elems;
        if (elems / (uint64_t)tg.qk > UINT64_MAX / (uint64_t)tg.bytes) return "GGUF tensor " + t.name + ": byte count overflows";
        t.nbytes = elems / (uint64_t)tg.qk * (uint64_t)tg.bytes;  // ggml_byte_len
        g->tensors.push_back(std::move(t));
    }
    g->data_start = ((uint64_t)r.pos + g->alignment - 1) / g->alignment * g->alignment;
    return "";
}

int fail(arfq_gguf *g, int status, const std::string &msg) {
    if (g) g->err = msg;
    g_gguf_err = msg;
    return status;
}

const arfq_gguf_tensor *find(const arfq_gguf *g, const char *name) {
    for (const auto &t : g->tensors)
        if (t.name == name) return &t;
    return nullptr;
}

// The tensor's bytes inside the mapping, or null when they run past its end.
const uint8_t *tensor_bytes(const arfq_gguf *g, const arfq_gguf_tensor &t) {
    const uint64_t base = g->data_start + t.offset;
    if (base < g->data_start || base > g->size || t.nbytes > g->size - base) return nullptr;
    return g->map + base;
}

}  // namespace

extern "C" {

int arfq_gguf_is_gguf(const char *path) {
    if (!path) return 0;
    struct stat st;
    if (stat(path, &st) != 0 || !S_ISREG(st.st_mode)) return 0;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return 0;
    char m[4];
    const ssize_t n = read(fd, m, 4);
    close(fd);
    return n == 4 && std::memcmp(m, "GGUF", 4) == 0;
}

int arfq_gguf_open(const char *path, arfq_gguf **out) {
    if (!out || !path) return fail(nullptr, ARFQ_E_INVALID, "arfq_gguf_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(nullptr, ARFQ_E_IO, std::string("arfq_gguf_open: cannot open ") + path + ": " + strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        close(fd);
        return fail(nullptr, ARFQ_E_IO, std::string("arfq_gguf_open: not a regular file: ") + path);
    }
    arfq_gguf *g = new (std::nothrow) arfq_gguf();
    if (!g) {
        close(fd);
        return fail(nullptr, ARFQ_E_NOMEM, "arfq_gguf_open: out of host memory");
    }
    g->size = (size_t)st.st_size;
    if (g->size) {
        void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            close(fd);
            delete g;
            return fail(nullptr, ARFQ_E_IO, std::string("arfq_gguf_open: mmap failed: ") + strerror(errno));
        }
        g->map = static_cast<const uint8_t *>(m);
    }
    close(fd);
    std::string e;
    try {
        e = parse(g);
    } catch (const std::exception &ex) {  // allocation failure on a huge table
        e = std::string("GGUF table: ") + ex.what();
    }
    if (!e.empty()) {
        arfq_gguf_close(g);
        return fail(nullptr, ARFQ_E_FORMAT, e);
    }
    *out = g;
    return ARFQ_OK;
}

int arfq_gguf_close(arfq_gguf *g) {
    if (!g) return ARFQ_E_INVALID;
    if (g->map) munmap(const_cast<uint8_t *>(g->map), g->size);
    delete g;
    return ARFQ_OK;
}

const char *arfq_gguf_last_error(const arfq_gguf *g) {
    return g ? g->err.c_str() : g_gguf_err.c_str();
}

int arfq_gguf_tensor_count(const arfq_gguf *g, int64_t *n) {
    if (!g || !n) return ARFQ_E_INVALID;
    *n = (int64_t)g->tensors.size();
    return ARFQ_OK;
}

int arfq_gguf_tensor_info(const arfq_gguf *g, int64_t index, const char **name, int *ggml_type,
                          int *n_dims, int64_t *dims, int max_dims, uint64_t *file_offset,
                          uint64_t *nbytes) {
    if (!g) return ARFQ_E_INVALID;
    if (index < 0 || index >= (int64_t)g->tensors.size())
        return fail(const_cast<arfq_gguf *>(g), ARFQ_E_INVALID, "arfq_gguf_tensor_info: index out of range");
    const arfq_gguf_tensor &t = g->tensors[(size_t)index];
    if (name) *name = t.name.c_str();
    if (ggml_type) *ggml_type = t.type;
    if (n_dims) *n_dims = (int)t.dims.size();
    if (dims)
        for (int d = 0; d < max_dims && d < (int)t.dims.size(); d++) dims[d] = (int64_t)t.dims[d];
    if (file_offset) *file_offset = g->data_start + t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return ARFQ_OK;
}

int arfq_gguf_find(const arfq_gguf *g, const char *name, int64_t *index) {
    if (!g || !name || !index) return ARFQ_E_INVALID;
    for (size_t i = 0; i < g->tensors.size(); i++)
        if (g->tensors[i].name == name) {
            *index = (int64_t)i;
            return ARFQ_OK;
        }
    return fail(const_cast<arfq_gguf *>(g), ARFQ_E_NOT_FOUND, std::string("no tensor named ") + name);
}

int arfq_gguf_blocks(const arfq_gguf *g, const char *name, int ggml_type, const void **blocks,
                     size_t *nbytes, int64_t *rows, int64_t *cols) {
    if (!g || !name) return ARFQ_E_INVALID;
    arfq_gguf *gm = const_cast<arfq_gguf *>(g);
    const arfq_gguf_tensor *t = find(g, name);
    if (!t) return fail(gm, ARFQ_E_NOT_FOUND, std::string("no tensor named ") + name);
    if (t->type != ggml_type)
        return fail(gm, ARFQ_E_UNSUPPORTED, "tensor " + t->name + " is ggml type " + std::to_string(t->type) +
                                                ", not " + std::to_string(ggml_type));
    const uint8_t *p = tensor_bytes(g, *t);
    if (!p) return fail(gm, ARFQ_E_FORMAT, "tensor " + t->name + ": data past the end of the file");
    const uint64_t c = t->dims.empty() ? 1 : t->dims[0];
    if (blocks) *blocks = p;
    if (nbytes) *nbytes = (size_t)t->nbytes;
    if (cols) *cols = (int64_t)c;
    if (rows) *rows = t->dims.size() >= 2 && c ? (int64_t)(t->elems / c) : 1;
    return ARFQ_OK;
}

int arfq_gguf_upload(arfq_ctx *ctx, const arfq_gguf *g, const char *name, int64_t row0, int64_t n_rows,
                     arfq_weight **out) {
    if (!ctx || !g || !name || !out) return ARFQ_E_INVALID;
    *out = nullptr;
    arfq_gguf *gm = const_cast<arfq_gguf *>(g);
    const arfq_gguf_tensor *t = find(g, name);
    if (!t) return fail(gm, ARFQ_E_NOT_FOUND, std::string("no tensor named ") + name);
    if (t->type != ARFQ_Q8_0 && t->type != ARFQ_Q4_K && t->type != ARFQ_Q6_K && t->type != ARFQ_Q5_K &&
        t->type != ARFQ_IQ4_XS)
        return fail(gm, ARFQ_E_UNSUPPORTED, "tensor " + t->name + ": ggml type " + std::to_string(t->type) +
                                                " has no matmul kernel here (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS)");
    const TypeGeom tg = type_geom(t->type);
    const uint8_t *p = tensor_bytes(g, *t);
    if (!p) return fail(gm, ARFQ_E_FORMAT, "tensor " + t->name + ": data past the end of the file");
    const size_t nd = t->dims.size();
    if (nd < 2 || nd > 3) return fail(gm, ARFQ_E_SHAPE, "tensor " + t->name + ": a matrix (2-D) or experts (3-D) expected");
    const uint64_t cols = t->dims[0], rows = t->dims[1], experts = nd == 3 ? t->dims[2] : 1;
    if (cols % (uint64_t)tg.qk)
        return fail(gm, ARFQ_E_SHAPE, "tensor " + t->name + ": row length " + std::to_string(cols) +
                                          " is not a whole number of blocks");
    if (cols > INT64_MAX / 2 || rows > INT64_MAX / 2 || experts > 65536)
        return fail(gm, ARFQ_E_SHAPE, "tensor " + t->name + ": dimensions out of range");
    const uint64_t row_bytes = cols / (uint64_t)tg.qk * (uint64_t)tg.bytes;
    if (nd == 3) {
        if (row0 != 0 || (n_rows >= 0 && (uint64_t)n_rows != rows))
            return fail(gm, ARFQ_E_SHAPE, "tensor " + t->name + ": row ranges apply to 2-D tensors only");
        return arfq_weight_upload(ctx, t->type, p, (size_t)t->nbytes, (int64_t)rows, (int64_t)cols, (int)experts, out);
    }
    const uint64_t nr = n_rows < 0 ? rows - (uint64_t)(row0 < 0 ? 0 : row0) : (uint64_t)n_rows;
    if (row0 < 0 || (uint64_t)row0 > rows || nr == 0 || nr > rows - (uint64_t)row0)
        return fail(gm, ARFQ_E_SHAPE, "tensor " + t->name + ": rows [" + std::to_string(row0) + ", +" +
                                          std::to_string(n_rows) + ") outside [0, " + std::to_string(rows) + ")");
    return arfq_weight_upload(ctx, t->type, p + (uint64_t)row0 * row_bytes, (size_t)(nr * row_bytes), (int64_t)nr,
                              (int64_t)cols, 1, out);
}

}  // extern "C"
