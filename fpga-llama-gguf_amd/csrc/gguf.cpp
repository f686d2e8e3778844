// GGUF reader (host only): parses the header, the key/value metadata and the tensor infos of a memory-mapped file.
// The layout is GGUF's published one: little-endian, strings as (u64 length, bytes), metadata values typed by a u32
// (0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array (u32 type, u64 count, values),
// 10 u64, 11 i64, 12 f64), tensor data aligned to general.alignment (default 32) after the infos.
#include "gemvq_gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <string>
#include <vector>

namespace {

thread_local std::string g_error;

struct Tensor {
    std::string name;
    int type = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0, nbytes = 0;
};

struct Value {
    bool numeric = false;
    double num = 0.0;
    std::string str;
};

// Bytes of a tensor of a ggml type (block types: block bytes per block elements).
bool type_size(int type, uint64_t & block_bytes, uint64_t & block_elems) {
    switch (type) {
    case 0: block_bytes = 4; block_elems = 1; return true;      // F32
    case 1: block_bytes = 2; block_elems = 1; return true;      // F16
    case 2: block_bytes = 18; block_elems = 32; return true;    // Q4_0
    case 3: block_bytes = 20; block_elems = 32; return true;    // Q4_1
    case 6: block_bytes = 22; block_elems = 32; return true;    // Q5_0
    case 7: block_bytes = 24; block_elems = 32; return true;    // Q5_1
    case 8: block_bytes = 34; block_elems = 32; return true;    // Q8_0
    case 10: block_bytes = 84; block_elems = 256; return true;  // Q2_K
    case 11: block_bytes = 110; block_elems = 256; return true; // Q3_K
    case 12: block_bytes = 144; block_elems = 256; return true; // Q4_K
    case 13: block_bytes = 176; block_elems = 256; return true; // Q5_K
    case 14: block_bytes = 210; block_elems = 256; return true; // Q6_K
    case 24: block_bytes = 1; block_elems = 1; return true;     // I8
    case 25: block_bytes = 2; block_elems = 1; return true;     // I16
    case 26: block_bytes = 4; block_elems = 1; return true;     // I32
    case 30: block_bytes = 2; block_elems = 1; return true;     // BF16
    default: return false;
    }
}

struct Cursor {
    const uint8_t * p;
    const uint8_t * end;
    bool ok = true;

    template <typename T>
    T get() {
        T v{};
        if (size_t(end - p) < sizeof(T)) {
            ok = false;
            return v;
        }
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > uint64_t(end - p)) {
            ok = false;
            return {};
        }
        std::string s(reinterpret_cast<const char *>(p), size_t(n));
        p += n;
        return s;
    }
    bool skip(uint64_t n) {
        if (n > uint64_t(end - p)) return ok = false;
        p += n;
        return true;
    }
};

size_t scalar_bytes(uint32_t t) {
    switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}

double scalar_value(uint32_t t, const uint8_t * p) {
    switch (t) {
    case 0: return *p;
    case 1: return int8_t(*p);
    case 7: return *p != 0;
    case 2: { uint16_t v; std::memcpy(&v, p, 2); return v; }
    case 3: { int16_t v; std::memcpy(&v, p, 2); return v; }
    case 4: { uint32_t v; std::memcpy(&v, p, 4); return v; }
    case 5: { int32_t v; std::memcpy(&v, p, 4); return v; }
    case 6: { float v; std::memcpy(&v, p, 4); return v; }
    case 10: { uint64_t v; std::memcpy(&v, p, 8); return double(v); }
    case 11: { int64_t v; std::memcpy(&v, p, 8); return double(v); }
    case 12: { double v; std::memcpy(&v, p, 8); return v; }
    default: return 0.0;
    }
}

}  // namespace

struct gemvq_gguf {
    int fd = -1;
    const uint8_t * base = nullptr;
    size_t size = 0;
    int version = 0;
    uint64_t data_start = 0;
    std::vector<Tensor> tensors;
    std::map<std::string, int> index;
    std::map<std::string, Value> kv;
};

extern "C" {

const char * gemvq_gguf_last_error(void) { return g_error.c_str(); }

void gemvq_gguf_close(gemvq_gguf * f) {
    if (!f) return;
    if (f->base) munmap(const_cast<uint8_t *>(f->base), f->size);
    if (f->fd >= 0) close(f->fd);
    delete f;
}

gemvq_gguf * gemvq_gguf_open(const char * path) {
    g_error.clear();
    if (!path) {
        g_error = "gguf: null path";
        return nullptr;
    }
    auto * f = new gemvq_gguf;
    f->fd = open(path, O_RDONLY);
    struct stat st {};
    if (f->fd < 0 || fstat(f->fd, &st) != 0 || st.st_size < 24) {
        g_error = std::string("gguf: cannot open or too small: ") + path;
        gemvq_gguf_close(f);
        return nullptr;
    }
    f->size = size_t(st.st_size);
    void * m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (m == MAP_FAILED) {
        g_error = "gguf: mmap failed";
        gemvq_gguf_close(f);
        return nullptr;
    }
    f->base = static_cast<const uint8_t *>(m);
    Cursor c{f->base, f->base + f->size};
    auto fail = [&](const std::string & why) -> gemvq_gguf * {
        g_error = "gguf: " + why;
        gemvq_gguf_close(f);
        return nullptr;
    };
    if (c.get<uint32_t>() != 0x46554747u) return fail("bad magic");
    f->version = int(c.get<uint32_t>());
    if (f->version != 2 && f->version != 3) return fail("unsupported version " + std::to_string(f->version));
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    if (!c.ok || n_tensors > (1u << 24) || n_kv > (1u << 24)) return fail("bad counts");
    for (uint64_t i = 0; i < n_kv && c.ok; ++i) {
        const std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        Value v;
        if (t == 8) {
            v.str = c.str();
        } else if (t == 9) {  // arrays (tokenizer tables and the like) are skipped, not kept
            const uint32_t et = c.get<uint32_t>();
            const uint64_t n = c.get<uint64_t>();
            if (et == 8) {
                for (uint64_t j = 0; j < n && c.ok; ++j) c.str();
            } else {
                const size_t eb = scalar_bytes(et);
                if (eb == 0 || n > uint64_t(c.end - c.p)) return fail("bad array in " + key);
                c.skip(n * eb);
            }
        } else {
            const size_t b = scalar_bytes(t);
            if (b == 0) return fail("bad value type in " + key);
            if (size_t(c.end - c.p) < b) return fail("truncated value " + key);
            v.numeric = true;
            v.num = scalar_value(t, c.p);
            c.skip(b);
        }
        if (c.ok && t != 9) f->kv[key] = v;
    }
    uint64_t align = 32;
    auto it = f->kv.find("general.alignment");
    if (it != f->kv.end() && it->second.numeric && it->second.num >= 1) align = uint64_t(it->second.num);
    for (uint64_t i = 0; i < n_tensors && c.ok; ++i) {
        Tensor t;
        t.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        if (nd > 4) return fail("tensor " + t.name + ": more than 4 dimensions");
        uint64_t elems = 1;
        for (uint32_t d = 0; d < nd; ++d) {
            t.ne[d] = int64_t(c.get<uint64_t>());
            if (t.ne[d] <= 0) return fail("tensor " + t.name + ": bad dimension");
            elems *= uint64_t(t.ne[d]);
        }
        t.type = int(c.get<uint32_t>());
        t.offset = c.get<uint64_t>();
        uint64_t bb = 0, be = 1;
        if (!type_size(t.type, bb, be)) return fail("tensor " + t.name + ": unsupported ggml type " + std::to_string(t.type));
        if (t.ne[0] % int64_t(be)) return fail("tensor " + t.name + ": row not a whole number of blocks");
        t.nbytes = elems / be * bb;
        f->index[t.name] = int(f->tensors.size());
        f->tensors.push_back(t);
    }
    if (!c.ok) return fail("truncated header");
    f->data_start = (uint64_t(c.p - f->base) + align - 1) / align * align;
    for (const Tensor & t : f->tensors)
        if (t.offset % align || f->data_start + t.offset + t.nbytes > f->size)
            return fail("tensor " + t.name + " lies outside the file or is misaligned");
    return f;
}

int gemvq_gguf_version(const gemvq_gguf * f) { return f ? f->version : -1; }
int gemvq_gguf_n_tensors(const gemvq_gguf * f) { return f ? int(f->tensors.size()) : -1; }

int gemvq_gguf_tensor(const gemvq_gguf * f, int i, char * name, size_t name_cap, int * type, int64_t ne[4],
                      const void ** data, uint64_t * nbytes) {
    if (!f || i < 0 || i >= int(f->tensors.size())) return -1;
    const Tensor & t = f->tensors[size_t(i)];
    if (name && name_cap) {
        const size_t n = std::min(name_cap - 1, t.name.size());
        std::memcpy(name, t.name.data(), n);
        name[n] = 0;
    }
    if (type) *type = t.type;
    if (ne)
        for (int d = 0; d < 4; ++d) ne[d] = t.ne[d];
    if (data) *data = f->base + f->data_start + t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return 0;
}

int64_t gemvq_gguf_file_offset(const gemvq_gguf * f, int i) {
    if (!f || i < 0 || i >= int(f->tensors.size())) return -1;
    return int64_t(f->data_start + f->tensors[size_t(i)].offset);
}

int gemvq_gguf_find(const gemvq_gguf * f, const char * name) {
    if (!f || !name) return -1;
    auto it = f->index.find(name);
    return it == f->index.end() ? -1 : it->second;
}

int gemvq_gguf_get_f64(const gemvq_gguf * f, const char * key, double * out) {
    if (!f || !key) return -1;
    auto it = f->kv.find(key);
    if (it == f->kv.end() || !it->second.numeric) return -1;
    if (out) *out = it->second.num;
    return 0;
}

const char * gemvq_gguf_get_str(const gemvq_gguf * f, const char * key) {
    if (!f || !key) return nullptr;
    auto it = f->kv.find(key);
    return (it == f->kv.end() || it->second.numeric) ? nullptr : it->second.str.c_str();
}

int gemvq_unrepack_q4_0x8(int rows, int cols, const void * x8, void * gguf_rows) {
    if (rows <= 0 || cols <= 0 || rows % 8 || cols % 32 || !x8 || !gguf_rows) return -1;
    constexpr size_t kX8 = 144, kQ4 = 18;
    constexpr uint64_t kFlip = 0x8888888888888888ull;  // x8 stores each nibble with its top bit flipped
    const size_t nb = size_t(cols) / 32, groups = size_t(rows) / 8;
    const auto * src = static_cast<const uint8_t *>(x8);
    auto * dst = static_cast<uint8_t *>(gguf_rows);
    for (size_t blk = 0; blk < groups * nb; ++blk) {  // x8 blocks in storage order: group-major, then column block
        const size_t g = blk / nb, b = blk % nb;
        const uint8_t * in = src + blk * kX8;
        uint8_t * row0 = dst + (g * 8 * nb + b) * kQ4;  // block b of the group's first row; rows are nb * kQ4 apart
        for (size_t c = 0; c < 16; ++c) {                // chunk c: quant bytes 8 (c / 8) .. + 7 of row c % 8
            uint64_t q;
            std::memcpy(&q, in + 16 + 8 * c, 8);
            q ^= kFlip;
            std::memcpy(row0 + (c % 8) * nb * kQ4 + 2 + 8 * (c / 8), &q, 8);
        }
        for (size_t r = 0; r < 8; ++r) std::memcpy(row0 + r * nb * kQ4, in + 2 * r, 2);  // the 8 fp16 scales
    }
    return 0;
}

}  // extern "C"
