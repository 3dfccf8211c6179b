// GGUF file reader and HBM upload (host code; no kernels).
//
// Behaviour of sycl-infer's reader (src/model/gguf.h, src/model/gguf.cpp):
//   - header: magic 'GGUF', version, n_tensors, n_kv, the kv pairs, then the
//     tensor infos; data section at the end of the infos rounded up to
//     general.alignment (32 by default); a tensor-less shard whose padding
//     runs past EOF gets data_offset = file size, a shard with tensors there
//     is "gguf: bad data offset" (gguf.cpp:240-289);
//   - kv values keep the reference's widening: integers in u64 and i64 with
//     the sign of their type, float32/float64 in f64, bool as 0/1, strings,
//     arrays of any element type (gguf.cpp:127-180); a key seen twice keeps
//     its last value;
//   - "name-0000i-of-0000n.gguf" names one shard of a split model: every
//     sibling is opened in index order, each is mapped at a page-aligned slot
//     of one PROT_NONE reservation so that (tensor data - map base) is one
//     offset space over the whole model, split.no / split.count are checked,
//     and the first shard that holds a key wins (gguf.cpp:308-456).
// Error messages are the reference's exception texts, returned through
// miq_last_error().
//
// MI355X side: miq_gguf_upload streams a byte range of the mapping into HBM
// through two pinned staging buffers, so the page-in of the next chunk runs
// while the DMA engine copies the previous one.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "../../include/miq.h"

namespace miq {
void set_error(const char *fmt, ...);
}

// A parsed kv value.  Arrays own their elements; `arr_type` keeps the element
// type even for an empty array.
struct miq_gguf_val {
    uint32_t type = 0;
    uint32_t arr_type = 0;
    uint64_t u64 = 0;
    int64_t i64 = 0;
    double f64 = 0;
    std::string str;
    std::vector<miq_gguf_val> arr;
};

namespace {

struct GgTensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
    const uint8_t *data = nullptr;
    int shard = 0;
};

struct GgShard {
    int fd = -1;
    uint8_t *base = nullptr;
    size_t size = 0;
    size_t data_offset = 0;
};

struct Header {
    uint32_t version = 0;
    size_t data_offset = 0;
    std::map<std::string, miq_gguf_val> kv;
    std::vector<GgTensor> tensors;
};

struct GgError {
    std::string what;
};

[[noreturn]] void fail(const std::string &what) { throw GgError{what}; }

// Bounds-checked little-endian cursor over one mapped shard.
struct Cursor {
    const uint8_t *p;
    const uint8_t *end;

    void need(uint64_t n) const {
        if (n > (uint64_t)(end - p)) fail("gguf: unexpected end of file");
    }
    template <typename T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        need(n);
        std::string s(reinterpret_cast<const char *>(p), (size_t)n);
        p += n;
        return s;
    }
    template <typename T>
    void integer(miq_gguf_val &v) {
        const T x = get<T>();
        if (T(-1) < T(0)) {  // signed: sign-extend into i64, u64 is its bit image
            v.i64 = (int64_t)x;
            v.u64 = (uint64_t)v.i64;
        } else {
            v.u64 = (uint64_t)x;
            v.i64 = (int64_t)v.u64;
        }
    }
    // GGUF value types 0..12 (uint8 int8 uint16 int16 uint32 int32 float32
    // bool string array uint64 int64 float64).
    void value(uint32_t type, miq_gguf_val &v, int depth) {
        v.type = type;
        switch (type) {
        case 0: integer<uint8_t>(v); break;
        case 1: integer<int8_t>(v); break;
        case 2: integer<uint16_t>(v); break;
        case 3: integer<int16_t>(v); break;
        case 4: integer<uint32_t>(v); break;
        case 5: integer<int32_t>(v); break;
        case 6: v.f64 = get<float>(); break;
        case 7: integer<uint8_t>(v); break;
        case 8: v.str = str(); break;
        case 9: {
            if (depth > 64) fail("gguf: arrays nested too deep");
            v.arr_type = get<uint32_t>();
            const uint64_t n = get<uint64_t>();
            need(n);  // every element takes at least one byte
            v.arr.resize((size_t)n);
            for (uint64_t i = 0; i < n; i++) value(v.arr_type, v.arr[i], depth + 1);
            v.u64 = n;
            break;
        }
        case 10: integer<uint64_t>(v); break;
        case 11: integer<int64_t>(v); break;
        case 12: v.f64 = get<double>(); break;
        default: fail("gguf: unknown kv type");
        }
    }
};

Header parse(const uint8_t *base, size_t size) {
    Cursor c{base, base + size};
    Header h;
    if (c.get<uint32_t>() != 0x46554747u) fail("not a gguf file");
    h.version = c.get<uint32_t>();
    const uint64_t n_tensors = c.get<uint64_t>();
    const uint64_t n_kv = c.get<uint64_t>();
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        miq_gguf_val v;
        c.value(t, v, 0);
        h.kv[key] = std::move(v);
    }
    c.need(n_tensors);  // a tensor info is at least 24 bytes
    h.tensors.resize((size_t)n_tensors);
    for (auto &t : h.tensors) {
        t.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        c.need((uint64_t)nd * 8);
        t.dims.resize(nd);
        for (auto &d : t.dims) d = c.get<uint64_t>();
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
    }
    uint64_t align = 32;
    auto it = h.kv.find("general.alignment");
    if (it != h.kv.end()) align = (uint32_t)it->second.u64;
    if (align == 0) fail("gguf: zero alignment");
    const uint64_t pos = (uint64_t)(c.p - base);
    uint64_t off = (pos + align - 1) / align * align;
    if (off > size) {
        if (n_tensors > 0) fail("gguf: bad data offset");
        off = size;  // metadata-only shard: no data section to point into
    }
    h.data_offset = (size_t)off;
    return h;
}

// Sibling paths of a split model named "...-IIIII-of-NNNNN.gguf", in index
// order; any other name is a single file.
std::vector<std::string> siblings(const std::string &path) {
    static const char kExt[] = ".gguf";
    const size_t ext = sizeof(kExt) - 1;
    if (path.size() < ext || path.compare(path.size() - ext, ext, kExt) != 0) return {path};
    const size_t of = path.rfind("-of-");
    if (of == std::string::npos || of < 6 || path.size() != of + 4 + 5 + ext) return {path};
    if (path[of - 6] != '-') return {path};
    const std::string idx = path.substr(of - 5, 5), cnt = path.substr(of + 4, 5);
    for (char ch : idx + cnt)
        if (ch < '0' || ch > '9') return {path};
    const int n = std::stoi(cnt);
    if (n <= 1) return {path};
    std::vector<std::string> out;
    const std::string stem = path.substr(0, of - 5);
    for (int i = 1; i <= n; i++) {
        char num[8];
        std::snprintf(num, sizeof(num), "%05d", i);
        out.push_back(stem + num + "-of-" + cnt + kExt);
    }
    return out;
}

int open_ro(const std::string &path, size_t *size) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) fail("cannot open " + path);
    struct stat st;
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        fail("fstat failed");
    }
    *size = (size_t)st.st_size;
    return fd;
}

uint64_t kv_u32(const Header &h, const char *key, uint64_t def) {
    auto it = h.kv.find(key);
    return it == h.kv.end() ? def : (uint32_t)it->second.u64;
}

size_t blck_size(uint32_t t) {
    switch (t) {
    case 0: case 1: case 30: return 1;                          // F32 F16 BF16
    case 2: case 3: case 6: case 7: case 8: case 9: case 20: return 32;  // Q4_0..Q8_1, IQ4_NL
    case 10: case 11: case 12: case 13: case 14: case 15:       // K-quants
    case 16: case 17: case 18: case 21: case 22: case 23: return 256;  // IQ2/IQ3/IQ4_XS
    default: return 0;
    }
}

size_t type_size(uint32_t t) {
    switch (t) {
    case 0: return 4;
    case 1: case 30: return 2;
    case 2: return 18;    // Q4_0: d + 16 B of nibbles
    case 3: return 20;    // Q4_1: d, m + 16
    case 6: return 22;    // Q5_0: d + 4 B high bits + 16
    case 7: return 24;    // Q5_1
    case 8: return 34;    // Q8_0: d + 32 codes
    case 9: return 36;    // Q8_1: d, s + 32
    case 10: return 84;   // Q2_K: d, dmin + 16 scales + 64
    case 11: return 110;  // Q3_K: 32 hmask + 64 + 12 scales + d
    case 12: return 144;  // Q4_K: d, dmin + 12 scales + 128
    case 13: return 176;  // Q5_K: + 32 B high bits
    case 14: return 210;  // Q6_K: 128 ql + 64 qh + 16 scales + d
    case 15: return 292;  // Q8_K: f32 d + 256 codes + 16 int16 bsums
    case 16: return 66;   // IQ2_XXS
    case 17: return 74;   // IQ2_XS
    case 18: return 98;   // IQ3_XXS
    case 20: return 18;   // IQ4_NL
    case 21: return 110;  // IQ3_S
    case 22: return 82;   // IQ2_S
    case 23: return 136;  // IQ4_XS
    default: return 0;
    }
}

size_t row_bytes(uint32_t t, uint64_t n) {
    const size_t bs = blck_size(t);
    if (bs == 0 || n % bs) return 0;
    return (size_t)(n / bs) * type_size(t);
}

}  // namespace

struct miq_gguf {
    uint8_t *map_base = nullptr;
    size_t map_size = 0;
    uint32_t version = 0;
    int split_count = 1;
    int split_no = 0;
    std::vector<GgShard> shards;
    std::vector<GgTensor> tensors;
    std::map<std::string, size_t> index;
    std::map<std::string, miq_gguf_val> kv;
    std::vector<const std::string *> keys;  // kv keys in sorted order
    // pinned staging for miq_gguf_upload (allocated on first use)
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    int stage_dev = -1;

    ~miq_gguf() {
        for (int i = 0; i < 2; i++) {
            if (done[i]) {
                (void)hipEventSynchronize(done[i]);
                (void)hipEventDestroy(done[i]);
            }
            if (stage[i]) (void)hipHostFree(stage[i]);
        }
        if (map_base) munmap(map_base, map_size);  // also drops the per-shard sub-mappings
        for (auto &s : shards)
            if (s.fd >= 0) ::close(s.fd);
    }

    void load(const std::string &path) {
        const std::vector<std::string> paths = siblings(path);
        const size_t page = (size_t)sysconf(_SC_PAGESIZE);
        std::vector<Header> hdr(paths.size());
        size_t total = 0;
        for (size_t i = 0; i < paths.size(); i++) {
            GgShard s;
            s.fd = open_ro(paths[i], &s.size);
            shards.push_back(s);
            if (s.size == 0) fail("mmap failed");
            // the header is parsed through a mapping of its own; the final
            // placement happens once every shard's size is known
            void *tmp = mmap(nullptr, s.size, PROT_READ, MAP_PRIVATE, s.fd, 0);
            if (tmp == MAP_FAILED) fail("mmap failed");
            try {
                hdr[i] = parse(static_cast<const uint8_t *>(tmp), s.size);
            } catch (...) {
                munmap(tmp, s.size);
                throw;
            }
            munmap(tmp, s.size);
            shards[i].data_offset = hdr[i].data_offset;
            total += (s.size + page - 1) / page * page;
            if (paths.size() > 1) {
                if (i == 0) {
                    split_count = (int)kv_u32(hdr[0], "split.count", paths.size());
                    split_no = (int)kv_u32(hdr[0], "split.no", 0);
                } else if ((int)kv_u32(hdr[i], "split.no", i) != (int)i) {
                    fail("gguf: shard " + paths[i] + " has split.no " +
                         std::to_string((int)kv_u32(hdr[i], "split.no", i)));
                }
                if ((int)kv_u32(hdr[i], "split.count", paths.size()) != (int)paths.size())
                    fail("gguf: split.count does not match the shard file names");
            }
        }
        version = hdr[0].version;
        for (auto &h : hdr)
            for (auto &e : h.kv) kv.emplace(e.first, e.second);  // first shard holding a key wins
        for (auto &e : kv) keys.push_back(&e.first);

        // one reservation, every shard at its page-aligned slot
        map_size = paths.size() == 1 ? shards[0].size : total;
        if (paths.size() == 1) {
            void *m = mmap(nullptr, map_size, PROT_READ, MAP_PRIVATE, shards[0].fd, 0);
            if (m == MAP_FAILED) fail("mmap failed");
            map_base = static_cast<uint8_t *>(m);
            shards[0].base = map_base;
        } else {
            void *m = mmap(nullptr, map_size, PROT_NONE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
            if (m == MAP_FAILED) fail("gguf: cannot reserve the split mapping");
            map_base = static_cast<uint8_t *>(m);
            size_t at = 0;
            for (size_t i = 0; i < paths.size(); i++) {
                const size_t slot = (shards[i].size + page - 1) / page * page;
                if (slot) {
                    void *p = mmap(map_base + at, slot, PROT_READ, MAP_PRIVATE | MAP_FIXED, shards[i].fd, 0);
                    if (p == MAP_FAILED) fail("gguf: cannot map shard " + paths[i]);
                }
                shards[i].base = map_base + at;
                at += slot;
            }
        }
        for (size_t i = 0; i < hdr.size(); i++) {
            for (auto &t : hdr[i].tensors) {
                t.data = shards[i].base + shards[i].data_offset + t.offset;
                t.shard = (int)i;
                index[t.name] = tensors.size();
                tensors.push_back(std::move(t));
            }
        }
    }

    // Reservation-relative ranges [lo, hi) that are file bytes (not the
    // padding after a shard's last page).
    template <typename F>
    void file_ranges(uint64_t off, uint64_t len, F &&f) const {
        for (size_t i = 0; i < shards.size(); i++) {
            const uint64_t s0 = (uint64_t)(shards[i].base - map_base), s1 = s0 + shards[i].size;
            const uint64_t lo = std::max(off, s0), hi = std::min(off + len, s1);
            if (hi > lo) f(i, lo, hi);
        }
    }
};

namespace {

constexpr size_t kStage = 32u << 20;  // pinned staging chunk

int upload(hipStream_t stream, miq_gguf *f, uint64_t off, uint64_t len, uint8_t *dst) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) {
        miq::set_error("miq_gguf_upload: no current device");
        return MIQ_EHIP;
    }
    if (f->stage_dev != dev) {
        // the events belong to the device current at their creation
        for (int i = 0; i < 2; i++) {
            if (f->done[i]) {
                (void)hipEventSynchronize(f->done[i]);
                (void)hipEventDestroy(f->done[i]);
                f->done[i] = nullptr;
            }
        }
        for (int i = 0; i < 2; i++) {
            if (!f->stage[i] && hipHostMalloc(&f->stage[i], kStage, hipHostMallocDefault) != hipSuccess) {
                f->stage[i] = nullptr;
                miq::set_error("miq_gguf_upload: hipHostMalloc(%zu) failed", kStage);
                return MIQ_EHIP;
            }
            if (hipEventCreateWithFlags(&f->done[i], hipEventDisableTiming) != hipSuccess) {
                f->done[i] = nullptr;
                miq::set_error("miq_gguf_upload: hipEventCreate failed");
                return MIQ_EHIP;
            }
        }
        f->stage_dev = dev;
    }
    uint64_t pos = 0;
    int b = 0;
    while (pos < len) {
        const uint64_t n = std::min<uint64_t>(kStage, len - pos);
        uint8_t *st = static_cast<uint8_t *>(f->stage[b]);
        if (hipEventSynchronize(f->done[b]) != hipSuccess) {
            miq::set_error("miq_gguf_upload: staging wait failed");
            return MIQ_EHIP;
        }
        // padding between shards reads as zero
        std::memset(st, 0, n);
        f->file_ranges(off + pos, n, [&](size_t, uint64_t lo, uint64_t hi) {
            std::memcpy(st + (lo - off - pos), f->map_base + lo, hi - lo);
        });
        if (hipMemcpyAsync(dst + pos, st, n, hipMemcpyHostToDevice, stream) != hipSuccess ||
            hipEventRecord(f->done[b], stream) != hipSuccess) {
            miq::set_error("miq_gguf_upload: hipMemcpyAsync failed");
            return MIQ_EHIP;
        }
        pos += n;
        b ^= 1;
    }
    for (int i = 0; i < 2; i++) {
        if (hipEventSynchronize(f->done[i]) != hipSuccess) {
            miq::set_error("miq_gguf_upload: copy failed");
            return MIQ_EHIP;
        }
    }
    return MIQ_OK;
}

void fill(const miq_gguf_val &v, miq_gguf_kv *out) {
    out->type = v.type;
    out->arr_type = v.arr_type;
    out->u64 = v.u64;
    out->i64 = v.i64;
    out->f64 = v.f64;
    out->str = v.type == 8 ? v.str.c_str() : nullptr;
    out->str_len = v.str.size();
    out->n = v.type == 9 ? (uint64_t)v.arr.size() : 0;
}

}  // namespace

extern "C" {

const char *miq_ggml_type_name(uint32_t t) {
    switch (t) {
    case 0: return "F32";
    case 1: return "F16";
    case 2: return "Q4_0";
    case 3: return "Q4_1";
    case 6: return "Q5_0";
    case 7: return "Q5_1";
    case 8: return "Q8_0";
    case 9: return "Q8_1";
    case 10: return "Q2_K";
    case 11: return "Q3_K";
    case 12: return "Q4_K";
    case 13: return "Q5_K";
    case 14: return "Q6_K";
    case 15: return "Q8_K";
    case 18: return "IQ3_XXS";
    case 20: return "IQ4_NL";
    case 21: return "IQ3_S";
    case 23: return "IQ4_XS";
    case 30: return "BF16";
    default: return "?";
    }
}

size_t miq_ggml_blck_size(uint32_t t) { return blck_size(t); }
size_t miq_ggml_type_size(uint32_t t) { return type_size(t); }
size_t miq_ggml_row_bytes(uint32_t t, uint64_t n) { return row_bytes(t, n); }

miq_gguf *miq_gguf_open(const char *path) {
    if (!path) {
        miq::set_error("miq_gguf_open: null path");
        return nullptr;
    }
    miq_gguf *f = new (std::nothrow) miq_gguf;
    if (!f) {
        miq::set_error("miq_gguf_open: out of memory");
        return nullptr;
    }
    try {
        f->load(path);
        return f;
    } catch (const GgError &e) {
        miq::set_error("%s", e.what.c_str());
    } catch (const std::exception &e) {
        miq::set_error("gguf: %s", e.what());
    }
    delete f;
    return nullptr;
}

void miq_gguf_close(miq_gguf *f) { delete f; }

int miq_gguf_describe(const miq_gguf *f, miq_gguf_desc *d) {
    if (!f || !d) return MIQ_EINVAL;
    d->version = f->version;
    d->n_tensors = (int64_t)f->tensors.size();
    d->n_kv = (int64_t)f->kv.size();
    d->n_shards = (int32_t)f->shards.size();
    d->split_count = f->split_count;
    d->split_no = f->split_no;
    d->map_base = f->map_base;
    d->map_size = f->map_size;
    d->data_offset = f->shards[0].data_offset;
    return MIQ_OK;
}

int miq_gguf_shard(const miq_gguf *f, int i, miq_gguf_shard_info *s) {
    if (!f || !s || i < 0 || i >= (int)f->shards.size()) return MIQ_EINVAL;
    s->base = f->shards[i].base;
    s->size = f->shards[i].size;
    s->data_offset = f->shards[i].data_offset;
    return MIQ_OK;
}

int64_t miq_gguf_find(const miq_gguf *f, const char *name) {
    if (!f || !name) return -1;
    auto it = f->index.find(name);
    return it == f->index.end() ? -1 : (int64_t)it->second;
}

int miq_gguf_tensor(const miq_gguf *f, int64_t i, miq_gguf_tensor_info *t) {
    if (!f || !t || i < 0 || i >= (int64_t)f->tensors.size()) return MIQ_EINVAL;
    const GgTensor &g = f->tensors[(size_t)i];
    t->name = g.name.c_str();
    t->type = g.type;
    t->n_dims = (uint32_t)g.dims.size();
    t->dims = g.dims.data();
    uint64_t ne = 1, rows = 1;
    for (size_t k = 0; k < g.dims.size(); k++) {
        ne *= g.dims[k];
        if (k) rows *= g.dims[k];
    }
    t->n_elements = ne;
    t->n_rows = rows;
    t->nbytes = row_bytes(g.type, ne);
    t->offset = g.offset;
    t->data = g.data;
    t->map_offset = (uint64_t)(g.data - f->map_base);
    t->shard = g.shard;
    return MIQ_OK;
}

const char *miq_gguf_kv_key(const miq_gguf *f, int64_t i) {
    if (!f || i < 0 || i >= (int64_t)f->keys.size()) return nullptr;
    return f->keys[(size_t)i]->c_str();
}

const miq_gguf_val *miq_gguf_meta(const miq_gguf *f, const char *key) {
    if (!f || !key) return nullptr;
    auto it = f->kv.find(key);
    return it == f->kv.end() ? nullptr : &it->second;
}

int miq_gguf_val_read(const miq_gguf_val *v, miq_gguf_kv *out) {
    if (!v || !out) return MIQ_EINVAL;
    fill(*v, out);
    return MIQ_OK;
}

const miq_gguf_val *miq_gguf_val_elem(const miq_gguf_val *v, uint64_t i) {
    if (!v || v->type != 9 || i >= v->arr.size()) return nullptr;
    return &v->arr[(size_t)i];
}

uint32_t miq_gguf_get_u32(const miq_gguf *f, const char *key, uint32_t def) {
    const miq_gguf_val *v = miq_gguf_meta(f, key);
    return v ? (uint32_t)v->u64 : def;
}

float miq_gguf_get_f32(const miq_gguf *f, const char *key, float def) {
    const miq_gguf_val *v = miq_gguf_meta(f, key);
    return v ? (float)v->f64 : def;
}

const char *miq_gguf_get_str(const miq_gguf *f, const char *key) {
    const miq_gguf_val *v = miq_gguf_meta(f, key);
    return v ? v->str.c_str() : nullptr;
}

int miq_gguf_drop_cache(const miq_gguf *f, uint64_t off, uint64_t len) {
    if (!f) return MIQ_EINVAL;
    f->file_ranges(off, len, [&](size_t i, uint64_t lo, uint64_t hi) {
        const uint64_t s0 = (uint64_t)(f->shards[i].base - f->map_base);
        (void)posix_fadvise(f->shards[i].fd, (off_t)(lo - s0), (off_t)(hi - lo), POSIX_FADV_DONTNEED);
    });
    return MIQ_OK;
}

int miq_gguf_upload(hipStream_t stream, miq_gguf *f, uint64_t off, uint64_t len, void *dst) {
    if (!f || !dst || off > f->map_size || len > f->map_size - off) {
        miq::set_error("miq_gguf_upload: bad arguments");
        return MIQ_EINVAL;
    }
    if (len == 0) return MIQ_OK;
    return upload(stream, f, off, len, static_cast<uint8_t *>(dst));
}

}  // extern "C"
