// GGUF v3 container reader (src/loader/gguf.rs) and the ggml dtype decoders
// (src/loader/dequant.rs), host side.
//
// The file is memory-mapped, never copied whole: the header, metadata and
// tensor table are parsed once into maps, and a tensor is decoded on request
// straight out of the mapping.  A Q4_0 tensor is not decoded at all: its
// 18-byte blocks {f16 d, 16 bytes of nibbles} are split into the scale image
// [N][K/32] f16 and the 16-byte-aligned quant image [N][K/32][16] that the
// decode GEMV streams (the same bytes, so the weights stay exactly the file's).
//
// Every read is bounds-checked: a truncated or inconsistent file is an error
// (CW_ERR_FORMAT), never an out-of-range access.  Decoding follows
// dequant.rs term by term: f32 products are rounded one at a time, no fused
// multiply-add (the pragma below), so each value equals the reference's
// Vec<f32> bit for bit.

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "cw_internal.hpp"

#pragma clang fp contract(off)

static_assert(__BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__, "GGUF is little-endian");

using cwi::set_error;

namespace {

enum MetaKind { META_OTHER, META_UINT, META_FLOAT, META_STRING };

// One metadata value, kept as gguf.rs's Meta enum keeps it (gguf.rs:14-21):
// every integer kind widened to u64 (signed ones sign-extended), f32/f64 as
// f64, strings as bytes, arrays as "other".
struct MetaValue {
    MetaKind kind = META_OTHER;
    uint64_t u = 0;
    double f = 0.0;
    std::string s;
};

struct TensorRec {
    uint32_t dtype = 0;
    std::vector<uint64_t> dims;  // ne[0] fastest (the "in" extent of a matrix)
    uint64_t n_elems = 0;
    uint64_t offset = 0;  // from the start of the data section
};

// Bounds-checked little-endian cursor over the mapped bytes.
struct Reader {
    const uint8_t *base;
    size_t size;
    size_t pos = 0;
    bool ok = true;

    const uint8_t *take(uint64_t n) {
        if (!ok || n > size - pos) {
            ok = false;
            return nullptr;
        }
        const uint8_t *p = base + pos;
        pos += n;
        return p;
    }
    template <class T>
    T get() {
        T v{};
        if (const uint8_t *p = take(sizeof(T))) std::memcpy(&v, p, sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        const uint8_t *p = take(n);
        return p ? std::string((const char *)p, n) : std::string();
    }
};

// Byte width of a fixed-size metadata scalar kind, 0 for string/array/unknown
// (gguf.rs:153-162).
int scalar_width(uint32_t kind) {
    switch (kind) {
        case 0: case 1: case 7: return 1;      // u8 i8 bool
        case 2: case 3: return 2;              // u16 i16
        case 4: case 5: case 6: return 4;      // u32 i32 f32
        case 10: case 11: case 12: return 8;   // u64 i64 f64
        default: return 0;
    }
}

// Skip `count` array elements of `kind`.  Nested arrays are walked as the
// GGUF format defines them (the reference skips none of their bytes, which
// desynchronises its cursor; real files carry no nested arrays).
bool skip_array(Reader &r, uint32_t kind, uint64_t count, int depth) {
    if (depth > 8) return false;
    if (const int w = scalar_width(kind)) {
        if (count > (r.size - r.pos) / (uint64_t)w) return false;
        r.take(count * (uint64_t)w);
        return r.ok;
    }
    for (uint64_t i = 0; i < count && r.ok; ++i) {
        if (kind == 8) {
            r.str();
        } else if (kind == 9) {
            const uint32_t k = r.get<uint32_t>();
            const uint64_t c = r.get<uint64_t>();
            if (!r.ok || !skip_array(r, k, c, depth + 1)) return false;
        } else {
            return false;
        }
    }
    return r.ok;
}

// read_meta_value (gguf.rs:125-151).  Returns false on an unknown kind.
bool read_meta(Reader &r, MetaValue &m) {
    const uint32_t kind = r.get<uint32_t>();
    switch (kind) {
        case 0: m.kind = META_UINT; m.u = r.get<uint8_t>(); break;
        case 1: m.kind = META_UINT; m.u = (uint64_t)(int64_t)r.get<int8_t>(); break;
        case 2: m.kind = META_UINT; m.u = r.get<uint16_t>(); break;
        case 3: m.kind = META_UINT; m.u = (uint64_t)(int64_t)r.get<int16_t>(); break;
        case 4: m.kind = META_UINT; m.u = r.get<uint32_t>(); break;
        case 5: m.kind = META_UINT; m.u = (uint64_t)(int64_t)r.get<int32_t>(); break;
        case 6: m.kind = META_FLOAT; m.f = (double)r.get<float>(); break;
        case 7: m.kind = META_UINT; m.u = r.get<uint8_t>(); break;
        case 8: m.kind = META_STRING; m.s = r.str(); break;
        case 9: {
            const uint32_t et = r.get<uint32_t>();
            const uint64_t count = r.get<uint64_t>();
            m.kind = META_OTHER;
            if (!r.ok || !skip_array(r, et, count, 0)) return false;
            break;
        }
        case 10: case 11: m.kind = META_UINT; m.u = r.get<uint64_t>(); break;
        case 12: m.kind = META_FLOAT; m.f = r.get<double>(); break;
        default: return false;
    }
    return r.ok;
}

// f16_to_f32 (dequant.rs:9-21): subnormals as mant * 2^-24, inf, and every
// NaN pattern to the canonical quiet NaN carrying the f16's sign.
inline float f16_value(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const int exp = (h >> 10) & 0x1f;
    const uint32_t mant = h & 0x3ff;
    float mag;
    if (exp == 0) {
        mag = (float)mant * 0x1p-24f;
    } else if (exp == 0x1f) {
        uint32_t bits = mant == 0 ? 0x7f800000u : 0x7fc00000u;
        std::memcpy(&mag, &bits, 4);
    } else {
        mag = std::ldexp(1.0f + (float)mant / 1024.0f, exp - 15);
    }
    uint32_t bits;
    std::memcpy(&bits, &mag, 4);
    bits |= sign;
    std::memcpy(&mag, &bits, 4);
    return mag;
}

inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// Elements per block and bytes per block of each decodable dtype
// (tensor_f32's dispatch, gguf.rs:109-122).
struct DtypeLayout {
    uint32_t qk, bytes;
};
bool dtype_layout(uint32_t dtype, DtypeLayout *l) {
    switch (dtype) {
        case CW_GGML_F32: *l = {1, 4}; return true;
        case CW_GGML_F16: *l = {1, 2}; return true;
        case CW_GGML_Q4_0: *l = {32, 18}; return true;
        case CW_GGML_Q4_1: *l = {32, 20}; return true;
        case CW_GGML_Q8_0: *l = {32, 34}; return true;
        case CW_GGML_Q6_K: *l = {256, 210}; return true;
        default: return false;
    }
}

// Decode blocks [lo, hi) of one dtype into out (block b -> out[b*qk ...]).
void decode_blocks(uint32_t dtype, const uint8_t *src, size_t lo, size_t hi, float *out) {
    switch (dtype) {
        case CW_GGML_F32:  // dequant_f32 (dequant.rs:31-35)
            std::memcpy(out + lo, src + lo * 4, (hi - lo) * 4);
            break;
        case CW_GGML_F16:  // dequant_f16 (dequant.rs:37-39)
            for (size_t i = lo; i < hi; ++i) out[i] = f16_value(rd16(src + 2 * i));
            break;
        case CW_GGML_Q4_0:  // dequant_q4_0 (dequant.rs:60-78)
            for (size_t b = lo; b < hi; ++b) {
                const uint8_t *p = src + b * 18;
                const float d = f16_value(rd16(p));
                float *y = out + b * 32;
                for (int j = 0; j < 16; ++j) {
                    y[j] = d * (float)((int)(p[2 + j] & 15) - 8);
                    y[j + 16] = d * (float)((int)(p[2 + j] >> 4) - 8);
                }
            }
            break;
        case CW_GGML_Q4_1:  // dequant_q4_1 (dequant.rs:80-97): d*q + m, no offset
            for (size_t b = lo; b < hi; ++b) {
                const uint8_t *p = src + b * 20;
                const float d = f16_value(rd16(p)), m = f16_value(rd16(p + 2));
                float *y = out + b * 32;
                for (int j = 0; j < 16; ++j) {
                    const float a = d * (float)(p[4 + j] & 15), c = d * (float)(p[4 + j] >> 4);
                    y[j] = a + m;
                    y[j + 16] = c + m;
                }
            }
            break;
        case CW_GGML_Q8_0:  // dequant_q8_0 (dequant.rs:44-56)
            for (size_t b = lo; b < hi; ++b) {
                const uint8_t *p = src + b * 34;
                const float d = f16_value(rd16(p));
                float *y = out + b * 32;
                for (int j = 0; j < 32; ++j) y[j] = d * (float)(int8_t)p[2 + j];
            }
            break;
        case CW_GGML_Q6_K:  // dequant_q6_k (dequant.rs:99-131), ggml's block_q6_K
            for (size_t b = lo; b < hi; ++b) {
                const uint8_t *ql = src + b * 210, *qh = ql + 128;
                const int8_t *sc = (const int8_t *)(ql + 192);
                const float d = f16_value(rd16(ql + 208));
                float *y = out + b * 256;
                // Each 128-element half: element 32*g + l (g = 0..3, l = 0..31)
                // takes its low 4 bits from ql[l + 32*(g&1)] (low nibble for
                // g < 2, high nibble otherwise), its top 2 bits from bits
                // 2g..2g+1 of qh[l], and the int8 scale sc[2g + l/16].
                for (int h = 0; h < 2; ++h) {
                    const uint8_t *L = ql + 64 * h, *H = qh + 32 * h;
                    const int8_t *S = sc + 8 * h;
                    float *Y = y + 128 * h;
                    for (int g = 0; g < 4; ++g) {
                        for (int l = 0; l < 32; ++l) {
                            const uint8_t byte = L[l + 32 * (g & 1)];
                            const int lo4 = g < 2 ? (byte & 15) : (byte >> 4);
                            const int q = (lo4 | (((H[l] >> (2 * g)) & 3) << 4)) - 32;
                            const float ds = d * (float)S[2 * g + l / 16];
                            Y[32 * g + l] = ds * (float)q;
                        }
                    }
                }
            }
            break;
        default:
            break;
    }
}

}  // namespace

struct cw_gguf {
    // the bytes: a private read-only mapping of the file, or an owned copy
    void *map = nullptr;
    size_t map_len = 0;
    std::vector<uint8_t> owned;
    const uint8_t *bytes = nullptr;
    size_t size = 0;

    uint32_t version = 0;
    std::unordered_map<std::string, MetaValue> meta;
    std::unordered_map<std::string, TensorRec> tensors;
    std::vector<std::string> order;  // tensor names in file order
    size_t data_start = 0;

    const TensorRec *find(const char *name) const {
        auto it = tensors.find(name);
        return it == tensors.end() ? nullptr : &it->second;
    }
};

namespace {

// GgufWeights::parse (gguf.rs:68-106) over g->bytes.
int parse_container(cw_gguf *g) {
    Reader r{g->bytes, g->size};
    const uint8_t *magic = r.take(4);
    if (!magic || std::memcmp(magic, "GGUF", 4) != 0) {
        set_error("not a GGUF file");
        return CW_ERR_FORMAT;
    }
    g->version = r.get<uint32_t>();
    const uint64_t n_tensors = r.get<uint64_t>();
    const uint64_t n_meta = r.get<uint64_t>();
    for (uint64_t i = 0; i < n_meta && r.ok; ++i) {
        std::string key = r.str();
        MetaValue v;
        const size_t at = r.pos;
        if (!r.ok) break;
        if (!read_meta(r, v)) {
            if (!r.ok) break;
            set_error("GGUF: bad metadata value for \"%s\" at byte %zu", key.c_str(), at);
            return CW_ERR_FORMAT;
        }
        g->meta[key] = std::move(v);  // a repeated key keeps the last value
    }
    for (uint64_t i = 0; i < n_tensors && r.ok; ++i) {
        std::string name = r.str();
        const uint32_t n_dims = r.get<uint32_t>();
        if (!r.ok || n_dims > 16) {
            set_error("GGUF: tensor \"%s\" has %u dims", name.c_str(), n_dims);
            return CW_ERR_FORMAT;
        }
        TensorRec t;
        t.n_elems = 1;
        for (uint32_t d = 0; d < n_dims; ++d) {
            const uint64_t e = r.get<uint64_t>();
            if (e != 0 && t.n_elems > UINT64_MAX / e) {
                set_error("GGUF: tensor \"%s\" element count overflows", name.c_str());
                return CW_ERR_FORMAT;
            }
            t.n_elems *= e;
            t.dims.push_back(e);
        }
        t.dtype = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        if (!r.ok) break;
        if (g->tensors.find(name) == g->tensors.end()) g->order.push_back(name);
        g->tensors[name] = std::move(t);  // a repeated name keeps the last entry
    }
    if (!r.ok) {
        set_error("GGUF: file truncated (%zu bytes) inside the header", g->size);
        return CW_ERR_FORMAT;
    }
    uint64_t align = 32;
    auto it = g->meta.find("general.alignment");
    if (it != g->meta.end() && it->second.kind == META_UINT) align = it->second.u;
    if (align == 0 || align > (1u << 30)) {
        set_error("GGUF: general.alignment = %llu", (unsigned long long)align);
        return CW_ERR_FORMAT;
    }
    const uint64_t start = (r.pos + align - 1) / align * align;
    if (start > g->size) {
        set_error("GGUF: data section starts at %llu, past the end of the file (%zu bytes)",
                  (unsigned long long)start, g->size);
        return CW_ERR_FORMAT;
    }
    g->data_start = (size_t)start;
    return CW_OK;
}

// The tensor's bytes, checked to lie inside the data section.
int tensor_bytes(const cw_gguf *g, const char *name, const TensorRec **out, const uint8_t **src,
                 DtypeLayout *lay) {
    const TensorRec *t = g->find(name);
    if (!t) {
        set_error("missing tensor %s", name);
        return CW_ERR_FORMAT;
    }
    if (!dtype_layout(t->dtype, lay)) {
        set_error("tensor %s: ggml dtype %u not supported yet", name, t->dtype);
        return CW_ERR_FORMAT;
    }
    if (t->n_elems % lay->qk != 0) {
        set_error("tensor %s: %llu elements is not a whole number of %u-element blocks", name,
                  (unsigned long long)t->n_elems, lay->qk);
        return CW_ERR_FORMAT;
    }
    const uint64_t n_blocks = t->n_elems / lay->qk;
    if (n_blocks > UINT64_MAX / lay->bytes) {
        set_error("tensor %s: %llu elements overflow its byte count", name,
                  (unsigned long long)t->n_elems);
        return CW_ERR_FORMAT;
    }
    const uint64_t nbytes = n_blocks * lay->bytes;
    const uint64_t avail = g->size - g->data_start;
    if (t->offset > avail || nbytes > avail - t->offset) {
        set_error("tensor %s: bytes [%llu, +%llu) run past the data section (%llu bytes)", name,
                  (unsigned long long)t->offset, (unsigned long long)nbytes,
                  (unsigned long long)avail);
        return CW_ERR_FORMAT;
    }
    *out = t;
    *src = g->bytes + g->data_start + t->offset;
    return CW_OK;
}

const MetaValue *meta_get(const cw_gguf *g, const char *key) {
    auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : &it->second;
}

// Rust's `f64 as u32`: truncate toward zero, saturate, NaN -> 0.
uint32_t f64_as_u32(double v) {
    if (!(v > 0.0)) return 0;
    if (v >= 4294967295.0) return 4294967295u;
    return (uint32_t)v;
}

uint32_t meta_u32_value(const cw_gguf *g, const char *key) {
    if (const MetaValue *m = meta_get(g, key)) {
        if (m->kind == META_UINT) return (uint32_t)m->u;
        if (m->kind == META_FLOAT) return f64_as_u32(m->f);
    }
    const size_t n = std::strlen(key);
    if (n >= 10 && std::strcmp(key + n - 10, "vocab_size") == 0) {
        if (const TensorRec *t = g->find("token_embd.weight")) {
            uint64_t mx = 0;
            for (uint64_t d : t->dims) mx = d > mx ? d : mx;
            return (uint32_t)mx;
        }
    }
    return 0;
}

}  // namespace

extern "C" {

int cw_gguf_open(const char *path, cw_gguf **out) {
    CW_CHECK_ARG(path && out, "cw_gguf_open: null argument");
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        set_error("cw_gguf_open: cannot open %s: %s", path, std::strerror(errno));
        return CW_ERR_IO;
    }
    struct stat st;
    if (fstat(fd, &st) != 0) {
        set_error("cw_gguf_open: cannot stat %s: %s", path, std::strerror(errno));
        ::close(fd);
        return CW_ERR_IO;
    }
    cw_gguf *g = new cw_gguf;
    g->size = (size_t)st.st_size;
    if (g->size > 0) {
        void *p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            set_error("cw_gguf_open: cannot map %s: %s", path, std::strerror(errno));
            ::close(fd);
            delete g;
            return CW_ERR_IO;
        }
        g->map = p;
        g->map_len = g->size;
        g->bytes = (const uint8_t *)p;
    }
    ::close(fd);
    const int rc = parse_container(g);
    if (rc != CW_OK) {
        cw_gguf_close(g);
        return rc;
    }
    *out = g;
    return CW_OK;
}

int cw_gguf_parse(const void *bytes, size_t len, cw_gguf **out) {
    CW_CHECK_ARG(out && (bytes || len == 0), "cw_gguf_parse: null argument");
    *out = nullptr;
    cw_gguf *g = new cw_gguf;
    g->owned.assign((const uint8_t *)bytes, (const uint8_t *)bytes + len);
    g->bytes = g->owned.data();
    g->size = len;
    const int rc = parse_container(g);
    if (rc != CW_OK) {
        delete g;
        return rc;
    }
    *out = g;
    return CW_OK;
}

int cw_gguf_close(cw_gguf *g) {
    if (!g) return CW_OK;
    if (g->map) munmap(g->map, g->map_len);
    delete g;
    return CW_OK;
}

int cw_gguf_info(const cw_gguf *g, uint32_t *version, uint64_t *n_tensors, uint64_t *n_meta,
                 uint64_t *data_offset) {
    CW_CHECK_ARG(g != nullptr, "cw_gguf_info: null handle");
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = g->order.size();
    if (n_meta) *n_meta = g->meta.size();
    if (data_offset) *data_offset = g->data_start;
    return CW_OK;
}

int cw_gguf_meta_u32(const cw_gguf *g, const char *key, uint32_t *out) {
    CW_CHECK_ARG(g && key && out, "cw_gguf_meta_u32: null argument");
    *out = meta_u32_value(g, key);
    return CW_OK;
}

int cw_gguf_meta_f32(const cw_gguf *g, const char *key, float *out) {
    CW_CHECK_ARG(g && key && out, "cw_gguf_meta_f32: null argument");
    const MetaValue *m = meta_get(g, key);
    *out = !m ? 0.0f
           : m->kind == META_FLOAT ? (float)m->f
           : m->kind == META_UINT  ? (float)m->u
                                   : 0.0f;
    return CW_OK;
}

int cw_gguf_meta_str(const cw_gguf *g, const char *key, char *buf, size_t buf_len,
                     size_t *len_out) {
    CW_CHECK_ARG(g && key, "cw_gguf_meta_str: null argument");
    const MetaValue *m = meta_get(g, key);
    if (!m || m->kind != META_STRING) {
        set_error("no string metadata \"%s\"", key);
        return CW_ERR_FORMAT;
    }
    if (len_out) *len_out = m->s.size();
    if (buf && buf_len > 0) {
        const size_t n = m->s.size() < buf_len - 1 ? m->s.size() : buf_len - 1;
        std::memcpy(buf, m->s.data(), n);
        buf[n] = 0;
    }
    return CW_OK;
}

int cw_gguf_has(const cw_gguf *g, const char *name) {
    return g && name && g->find(name) ? 1 : 0;
}

int cw_gguf_tensor_name(const cw_gguf *g, uint64_t index, char *buf, size_t buf_len) {
    CW_CHECK_ARG(g && buf && buf_len > 0, "cw_gguf_tensor_name: null argument");
    CW_CHECK_ARG(index < g->order.size(), "cw_gguf_tensor_name: index %llu of %zu",
                 (unsigned long long)index, g->order.size());
    const std::string &s = g->order[index];
    CW_CHECK_ARG(s.size() < buf_len, "cw_gguf_tensor_name: name needs %zu bytes", s.size() + 1);
    std::memcpy(buf, s.c_str(), s.size() + 1);
    return CW_OK;
}

int cw_gguf_tensor_info(const cw_gguf *g, const char *name, uint32_t *dtype, int *n_dims,
                        uint64_t *dims, int max_dims, uint64_t *n_elems, uint64_t *offset) {
    CW_CHECK_ARG(g && name, "cw_gguf_tensor_info: null argument");
    const TensorRec *t = g->find(name);
    if (!t) {
        set_error("missing tensor %s", name);
        return CW_ERR_FORMAT;
    }
    if (dtype) *dtype = t->dtype;
    if (n_dims) *n_dims = (int)t->dims.size();
    if (dims)
        for (int i = 0; i < max_dims && i < (int)t->dims.size(); ++i) dims[i] = t->dims[i];
    if (n_elems) *n_elems = t->n_elems;
    if (offset) *offset = t->offset;
    return CW_OK;
}

int cw_gguf_tensor_f32(const cw_gguf *g, const char *name, float *out, size_t n) {
    CW_CHECK_ARG(g && name && out, "cw_gguf_tensor_f32: null argument");
    const TensorRec *t = nullptr;
    const uint8_t *src = nullptr;
    DtypeLayout lay{};
    CW_TRY(tensor_bytes(g, name, &t, &src, &lay));
    CW_CHECK_ARG(n == t->n_elems, "cw_gguf_tensor_f32: %s has %llu elements, buffer holds %zu",
                 name, (unsigned long long)t->n_elems, n);
    const size_t units = lay.qk == 1 ? n : n / lay.qk;
    cwi::parallel_for(units, [&](size_t lo, size_t hi) { decode_blocks(t->dtype, src, lo, hi, out); });
    return CW_OK;
}

int cw_gguf_tensor_q4(const cw_gguf *g, const char *name, size_t out_f, size_t in_f,
                      uint16_t *scales, uint8_t *quants) {
    CW_CHECK_ARG(g && name && scales && quants, "cw_gguf_tensor_q4: null argument");
    CW_CHECK_ARG(in_f > 0 && in_f % 32 == 0, "cw_gguf_tensor_q4: in_f=%zu must be a multiple of 32",
                 in_f);
    const TensorRec *t = nullptr;
    const uint8_t *src = nullptr;
    DtypeLayout lay{};
    CW_TRY(tensor_bytes(g, name, &t, &src, &lay));
    if (t->n_elems != (uint64_t)out_f * in_f || (!t->dims.empty() && t->dims[0] != in_f)) {
        set_error("tensor %s: shape (ne0=%llu, %llu elements) is not [%zu][%zu]", name,
                  (unsigned long long)(t->dims.empty() ? 0 : t->dims[0]),
                  (unsigned long long)t->n_elems, out_f, in_f);
        return CW_ERR_FORMAT;
    }
    const size_t nblk = out_f * (in_f / 32);
    if (t->dtype == CW_GGML_Q4_0) {
        // the file's blocks, split: no decode, no requantization
        cwi::parallel_for(nblk, [&](size_t lo, size_t hi) {
            for (size_t b = lo; b < hi; ++b) {
                const uint8_t *p = src + b * 18;
                scales[b] = rd16(p);
                std::memcpy(quants + b * 16, p + 2, 16);
            }
        });
        return CW_OK;
    }
    // any other dtype: decode to f32, then the Q4_0 quantizer (the path the
    // reference's Proj::load takes for every projection under --quantize)
    std::vector<float> f((size_t)t->n_elems);
    CW_TRY(cw_gguf_tensor_f32(g, name, f.data(), f.size()));
    return cw_q4_quantize(f.data(), out_f, in_f, scales, quants);
}

int cw_gguf_model_config(const cw_gguf *g, int max_seq, int kv_dtype, cw_model_config *cfg) {
    CW_CHECK_ARG(g && cfg, "cw_gguf_model_config: null argument");
    CW_CHECK_ARG(max_seq > 0, "cw_gguf_model_config: max_seq=%d", max_seq);
    CW_CHECK_ARG(kv_dtype == CW_F32 || kv_dtype == CW_F16, "cw_gguf_model_config: kv_dtype=%d",
                 kv_dtype);
    if (const MetaValue *a = meta_get(g, "general.architecture")) {
        if (a->kind == META_STRING && a->s != "qwen3") {
            set_error("GGUF architecture \"%s\": only qwen3 is built", a->s.c_str());
            return CW_ERR_FORMAT;
        }
    }
    // the keys Qwen3::load reads (qwen3.rs:44-53)
    const char *ukeys[] = {"qwen3.block_count", "qwen3.embedding_length",
                           "qwen3.attention.head_count", "qwen3.attention.head_count_kv",
                           "qwen3.attention.key_length", "qwen3.feed_forward_length",
                           "qwen3.vocab_size"};
    int *dst[] = {&cfg->n_layers, &cfg->dim, &cfg->n_heads, &cfg->n_kv_heads,
                  &cfg->head_dim, &cfg->hidden, &cfg->vocab};
    for (int i = 0; i < 7; ++i) {
        const uint32_t v = meta_u32_value(g, ukeys[i]);
        if (v == 0 || v > (uint32_t)INT32_MAX) {
            set_error("GGUF: metadata %s is missing or out of range (%u)", ukeys[i], v);
            return CW_ERR_FORMAT;
        }
        *dst[i] = (int)v;
    }
    CW_TRY(cw_gguf_meta_f32(g, "qwen3.attention.layer_norm_rms_epsilon", &cfg->eps));
    CW_TRY(cw_gguf_meta_f32(g, "qwen3.rope.freq_base", &cfg->rope_theta));
    cfg->family = cw_family_spec{0, 0, 1, 0};
    cfg->max_seq = max_seq;
    cfg->kv_dtype = kv_dtype;
    return CW_OK;
}

}  // extern "C"
