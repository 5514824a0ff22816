// The weight path feeding the linears: a memory-mapped .safetensors file, and the
// 256-byte-aligned device arena of one module's 16-bit weights.
//
// Reference: SafeTensors (SafeTensors.swift:7-87) and WeightArena (Weights.swift:8-79).
//   - The file is an 8-byte little-endian header length, a JSON header {name: {dtype, shape,
//     data_offsets: [begin, end]}, "__metadata__": {...}}, then the data; offsets are relative
//     to the end of the header.  Malformed headers and files shorter than the header claims
//     are refused with the reference's messages.
//   - The arena places tensors at 256-byte-aligned offsets in call order; a tensor may be the
//     concatenation of several bf16 tensors along their first axis (q, k, v rows), or a
//     [n, stored_k] weight laid out as [n, k] with zero columns past stored_k.
// MI355X side: the plan is recorded first and the caller allocates the device arena (the
// reference sizes and then copies in two passes of the same builder); the upload moves the
// mapped bytes through two pinned staging buffers with asynchronous copies, so the copy of
// one buffer overlaps the host fill of the other; an optional in-place kernel converts the
// bf16 weights to fp16 (round to nearest even) and counts the values that overflow to +-inf
// and the nonzero values that flush to zero.
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <map>
#include <string>
#include <vector>

#include "mt_device.hpp"
#include "mt_internal.hpp"
#include "mingtts_hip.h"

namespace mt {

namespace {

// ---------------------------------------------------------------- header JSON --

struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0;
    bool neg = false;
    uint64_t u = 0;      // the number when it is a non-negative integer
    bool integer = false;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
};

class Parser {
  public:
    Parser(const char *p, size_t n) : p_(p), end_(p + n) {}
    bool parse(Json &out) {
        ws();
        if (!value(out, 0)) return false;
        ws();
        return p_ == end_;
    }

  private:
    const char *p_, *end_;
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    bool lit(const char *s) {
        const size_t n = strlen(s);
        if (static_cast<size_t>(end_ - p_) < n || memcmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    bool string(std::string &s) {
        if (p_ >= end_ || *p_ != '"') return false;
        p_++;
        while (p_ < end_ && *p_ != '"') {
            if (*p_ == '\\') {
                if (++p_ >= end_) return false;
                const char c = *p_++;
                switch (c) {
                    case '"': s += '"'; break;
                    case '\\': s += '\\'; break;
                    case '/': s += '/'; break;
                    case 'b': s += '\b'; break;
                    case 'f': s += '\f'; break;
                    case 'n': s += '\n'; break;
                    case 'r': s += '\r'; break;
                    case 't': s += '\t'; break;
                    case 'u': {
                        if (end_ - p_ < 4) return false;
                        unsigned v = 0;
                        for (int i = 0; i < 4; i++) {
                            const char h = *p_++;
                            v <<= 4;
                            if (h >= '0' && h <= '9') v |= h - '0';
                            else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
                            else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
                            else return false;
                        }
                        if (v < 0x80) s += static_cast<char>(v);  // names are ASCII; others kept as UTF-8
                        else if (v < 0x800) { s += static_cast<char>(0xC0 | (v >> 6)); s += static_cast<char>(0x80 | (v & 0x3F)); }
                        else { s += static_cast<char>(0xE0 | (v >> 12)); s += static_cast<char>(0x80 | ((v >> 6) & 0x3F)); s += static_cast<char>(0x80 | (v & 0x3F)); }
                        break;
                    }
                    default: return false;
                }
            } else {
                s += *p_++;
            }
        }
        if (p_ >= end_) return false;
        p_++;
        return true;
    }
    bool number(Json &j) {
        const char *b = p_;
        if (p_ < end_ && *p_ == '-') { j.neg = true; p_++; }
        if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
        bool frac = false;
        while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' || *p_ == '-')) {
            if (*p_ == '.' || *p_ == 'e' || *p_ == 'E') frac = true;
            p_++;
        }
        const std::string t(b, p_);
        j.kind = Json::NUM;
        j.num = strtod(t.c_str(), nullptr);
        j.integer = !frac && !j.neg && t.size() <= 19;
        if (j.integer) j.u = strtoull(t.c_str(), nullptr, 10);
        return true;
    }
    bool value(Json &j, int depth) {
        if (depth > 16 || p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            p_++;
            j.kind = Json::OBJ;
            ws();
            if (p_ < end_ && *p_ == '}') { p_++; return true; }
            for (;;) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (p_ >= end_ || *p_++ != ':') return false;
                ws();
                Json v;
                if (!value(v, depth + 1)) return false;
                j.obj.emplace_back(std::move(k), std::move(v));
                ws();
                if (p_ < end_ && *p_ == ',') { p_++; continue; }
                if (p_ < end_ && *p_ == '}') { p_++; return true; }
                return false;
            }
        }
        if (c == '[') {
            p_++;
            j.kind = Json::ARR;
            ws();
            if (p_ < end_ && *p_ == ']') { p_++; return true; }
            for (;;) {
                ws();
                Json v;
                if (!value(v, depth + 1)) return false;
                j.arr.push_back(std::move(v));
                ws();
                if (p_ < end_ && *p_ == ',') { p_++; continue; }
                if (p_ < end_ && *p_ == ']') { p_++; return true; }
                return false;
            }
        }
        if (c == '"') { j.kind = Json::STR; return string(j.str); }
        if (lit("true")) { j.kind = Json::BOOL; return true; }
        if (lit("false")) { j.kind = Json::BOOL; return true; }
        if (lit("null")) { j.kind = Json::NUL; return true; }
        return number(j);
    }
};

const Json *field(const Json &o, const char *k) {
    for (const auto &kv : o.obj)
        if (kv.first == k) return &kv.second;
    return nullptr;
}

int dtype_code(const std::string &d) {
    if (d == "BF16") return MT_BF16;
    if (d == "F16") return MT_F16;
    if (d == "F32") return MT_F32;
    return -1;
}

}  // namespace

struct StFile {
    struct Entry {
        std::string dtype;
        std::vector<uint64_t> shape;
        uint64_t begin = 0, end = 0;
    };
    void *map = nullptr;
    size_t size = 0;
    uint64_t data_start = 0;
    std::vector<std::string> names;  // header order
    std::map<std::string, Entry> entries;
};

// One planned piece of the arena: bytes from the file to a device offset, or a padded
// weight copied row by row.
struct ArenaCopy {
    uint64_t dst;
    const uint8_t *src;
    uint64_t bytes;      // plain copy
    uint32_t rows = 0;   // padded: rows of src_row bytes placed at dst_row strides
    uint64_t src_row = 0, dst_row = 0;
};

struct Arena {
    const StFile *st = nullptr;
    int convert_to = MT_BF16;
    uint64_t cursor = 0;
    std::vector<ArenaCopy> copies;
    uint64_t overflow = 0, underflow = 0;
    bool uploaded = false;
};

namespace {

uint64_t place(Arena &a, uint64_t bytes) {
    const uint64_t off = a.cursor;
    a.cursor += (bytes + 255) & ~uint64_t(255);
    return off;
}

// In-place bf16 -> fp16 (round to nearest even), counting finite values that become +-inf
// and nonzero values that become zero.  Eight elements per thread per step, grid-stride.
__global__ __launch_bounds__(256) void bf16_to_f16_kernel(uint16_t *p, uint64_t n8, unsigned long long *counts) {
    unsigned long long ov = 0, un = 0;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n8; i += static_cast<uint64_t>(gridDim.x) * 256ull) {
        uint4 v = reinterpret_cast<uint4 *>(p)[i];
        uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            uint32_t out = 0;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint16_t b = static_cast<uint16_t>(w[e] >> (16 * h));
                const float f = __uint_as_float(static_cast<uint32_t>(b) << 16);
                const _Float16 x = static_cast<_Float16>(f);
                const uint16_t xb = __builtin_bit_cast(uint16_t, x);
                const bool finite = (b & 0x7F80u) != 0x7F80u;
                ov += finite && (xb & 0x7FFFu) == 0x7C00u;
                un += (b & 0x7FFFu) != 0 && (xb & 0x7FFFu) == 0;
                out |= static_cast<uint32_t>(xb) << (16 * h);
            }
            w[e] = out;
        }
        reinterpret_cast<uint4 *>(p)[i] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    for (int off = 32; off > 0; off >>= 1) {
        ov += __shfl_xor(ov, off, 64);
        un += __shfl_xor(un, off, 64);
    }
    if ((threadIdx.x & 63) == 0 && (ov || un)) {
        atomicAdd(counts, ov);
        atomicAdd(counts + 1, un);
    }
}

}  // namespace

}  // namespace mt

using namespace mt;

extern "C" {

int mt_st_open(const char *path, mt_st **out) {
    if (!out || !path) return set_error(MT_EINVAL, "mt_st_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return set_error(MT_EINVAL, "mt_st_open: cannot open %s", path);
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        close(fd);
        return set_error(MT_EINVAL, "mt_st_open: cannot stat %s", path);
    }
    const size_t size = static_cast<size_t>(sb.st_size);
    if (size < 8) {
        close(fd);
        return set_error(MT_EINVAL, "bad checkpoint: file too small");
    }
    void *map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return set_error(MT_EINVAL, "mt_st_open: cannot map %s", path);
    StFile *f = new StFile();
    f->map = map;
    f->size = size;
    auto fail = [&](int rc) {
        munmap(map, size);
        delete f;
        return rc;
    };
    uint64_t hl = 0;
    memcpy(&hl, map, 8);  // little-endian, as the format and the host are
    if (hl == 0 || hl > size - 8)
        return fail(set_error(MT_EINVAL, "bad checkpoint: header length %llu exceeds file",
                              static_cast<unsigned long long>(hl)));
    Json j;
    if (!Parser(static_cast<const char *>(map) + 8, hl).parse(j) || j.kind != Json::OBJ)
        return fail(set_error(MT_EINVAL, "bad checkpoint: header is not a JSON object"));
    f->data_start = 8 + hl;
    uint64_t last = 0;
    for (const auto &kv : j.obj) {
        if (kv.first == "__metadata__") continue;
        const Json *dt = kv.second.kind == Json::OBJ ? field(kv.second, "dtype") : nullptr;
        const Json *sh = kv.second.kind == Json::OBJ ? field(kv.second, "shape") : nullptr;
        const Json *of = kv.second.kind == Json::OBJ ? field(kv.second, "data_offsets") : nullptr;
        bool ok = dt && dt->kind == Json::STR && sh && sh->kind == Json::ARR && of && of->kind == Json::ARR &&
                  of->arr.size() == 2 && of->arr[0].integer && of->arr[1].integer && of->arr[0].u <= of->arr[1].u;
        StFile::Entry e;
        if (ok) {
            for (const Json &d : sh->arr) {
                if (!d.integer) { ok = false; break; }
                e.shape.push_back(d.u);
            }
        }
        if (!ok || f->entries.count(kv.first))
            return fail(set_error(MT_EINVAL, "bad checkpoint: malformed entry %s", kv.first.c_str()));
        e.dtype = dt->str;
        e.begin = of->arr[0].u;
        e.end = of->arr[1].u;
        last = std::max(last, e.end);
        f->names.push_back(kv.first);
        f->entries.emplace(kv.first, std::move(e));
    }
    if (f->data_start + last > size)
        return fail(set_error(MT_EINVAL, "bad checkpoint: file holds %llu bytes, header needs %llu; download incomplete?",
                              static_cast<unsigned long long>(size), static_cast<unsigned long long>(f->data_start + last)));
    *out = reinterpret_cast<mt_st *>(f);
    return MT_OK;
}

int mt_st_close(mt_st *st) {
    StFile *f = reinterpret_cast<StFile *>(st);
    if (!f) return MT_OK;
    munmap(f->map, f->size);
    delete f;
    return MT_OK;
}

int mt_st_count(const mt_st *st) {
    if (!st) return set_error(MT_EINVAL, "mt_st_count: null file");
    return static_cast<int>(reinterpret_cast<const StFile *>(st)->names.size());
}

int mt_st_name(const mt_st *st, uint32_t index, const char **name) {
    const StFile *f = reinterpret_cast<const StFile *>(st);
    if (!f || !name) return set_error(MT_EINVAL, "mt_st_name: null argument");
    if (index >= f->names.size()) return set_error(MT_EINVAL, "mt_st_name: index %u out of range", index);
    *name = f->names[index].c_str();
    return MT_OK;
}

int mt_st_find(const mt_st *st, const char *name, mt_st_entry *out) {
    const StFile *f = reinterpret_cast<const StFile *>(st);
    if (!f || !name || !out) return set_error(MT_EINVAL, "mt_st_find: null argument");
    auto it = f->entries.find(name);
    if (it == f->entries.end()) return set_error(MT_EINVAL, "missing tensor %s", name);
    const StFile::Entry &e = it->second;
    memset(out, 0, sizeof(*out));
    out->dtype = dtype_code(e.dtype);
    out->ndim = static_cast<uint32_t>(std::min<size_t>(e.shape.size(), 8));
    for (uint32_t i = 0; i < out->ndim; i++) out->shape[i] = e.shape[i];
    out->bytes = e.end - e.begin;
    out->host = static_cast<const uint8_t *>(f->map) + f->data_start + e.begin;
    return MT_OK;
}

int mt_arena_create(const mt_st *st, mt_dtype convert_to, mt_arena **out) {
    if (!st || !out) return set_error(MT_EINVAL, "mt_arena_create: null argument");
    if (convert_to != MT_BF16 && convert_to != MT_F16)
        return set_error(MT_EINVAL, "mt_arena_create: the arena holds MT_BF16 (as stored) or MT_F16 (converted)");
    Arena *a = new Arena();
    a->st = reinterpret_cast<const StFile *>(st);
    a->convert_to = convert_to;
    *out = reinterpret_cast<mt_arena *>(a);
    return MT_OK;
}

// Does a BF16 entry's byte range hold exactly its shape's elements?  (A header whose shape
// claims more than its data_offsets span would make the copies read past the tensor.)
static bool bf16_bytes_match(const StFile::Entry &e) {
    uint64_t elems = 1;
    for (uint64_t d : e.shape) {
        if (d != 0 && elems > UINT64_MAX / 2 / d) return false;
        elems *= d;
    }
    return e.end - e.begin == elems * 2;
}

int mt_arena_tensor(mt_arena *arena, const char *const *names, uint32_t n_names, uint64_t *offset, uint64_t *count) {
    Arena *a = reinterpret_cast<Arena *>(arena);
    if (!a || !names || n_names == 0 || !offset) return set_error(MT_EINVAL, "mt_arena_tensor: null argument");
    if (a->uploaded) return set_error(MT_EINVAL, "mt_arena_tensor: the arena is already uploaded");
    uint64_t total = 0;
    std::vector<const StFile::Entry *> es;
    for (uint32_t i = 0; i < n_names; i++) {
        if (!names[i]) return set_error(MT_EINVAL, "mt_arena_tensor: null name");
        auto it = a->st->entries.find(names[i]);
        if (it == a->st->entries.end()) return set_error(MT_EINVAL, "missing tensor %s", names[i]);
        if (it->second.dtype != "BF16")
            return set_error(MT_EINVAL, "bad checkpoint: %s is %s, expected BF16", names[i], it->second.dtype.c_str());
        if (!bf16_bytes_match(it->second))
            return set_error(MT_EINVAL, "bad checkpoint: %s: data_offsets span %llu bytes, its shape needs another count",
                             names[i], static_cast<unsigned long long>(it->second.end - it->second.begin));
        es.push_back(&it->second);
        total += it->second.end - it->second.begin;
    }
    const uint64_t off = place(*a, total);
    uint64_t dst = off;
    for (const StFile::Entry *e : es) {
        ArenaCopy c;
        c.dst = dst;
        c.src = static_cast<const uint8_t *>(a->st->map) + a->st->data_start + e->begin;
        c.bytes = e->end - e->begin;
        a->copies.push_back(c);
        dst += c.bytes;
    }
    *offset = off;
    if (count) *count = total / 2;
    return MT_OK;
}

int mt_arena_padded(mt_arena *arena, const char *name, uint32_t n, uint32_t k, uint32_t stored_k, uint64_t *offset) {
    Arena *a = reinterpret_cast<Arena *>(arena);
    if (!a || !name || !offset) return set_error(MT_EINVAL, "mt_arena_padded: null argument");
    if (a->uploaded) return set_error(MT_EINVAL, "mt_arena_padded: the arena is already uploaded");
    auto it = a->st->entries.find(name);
    if (it == a->st->entries.end()) return set_error(MT_EINVAL, "missing tensor %s", name);
    const StFile::Entry &e = it->second;
    if (e.dtype != "BF16" || e.shape.size() != 2 || e.shape[0] != n || e.shape[1] != stored_k || stored_k > k)
        return set_error(MT_EINVAL, "bad checkpoint: %s is not BF16 [%u, %u] (or k %u < stored k)", name, n, stored_k, k);
    if (!bf16_bytes_match(e))
        return set_error(MT_EINVAL, "bad checkpoint: %s: data_offsets span %llu bytes, its shape [%u, %u] needs %llu",
                         name, static_cast<unsigned long long>(e.end - e.begin), n, stored_k,
                         static_cast<unsigned long long>(n) * stored_k * 2);
    const uint64_t off = place(*a, static_cast<uint64_t>(n) * k * 2);
    ArenaCopy c;
    c.dst = off;
    c.src = static_cast<const uint8_t *>(a->st->map) + a->st->data_start + e.begin;
    c.bytes = static_cast<uint64_t>(n) * k * 2;
    c.rows = n;
    c.src_row = static_cast<uint64_t>(stored_k) * 2;
    c.dst_row = static_cast<uint64_t>(k) * 2;
    a->copies.push_back(c);
    *offset = off;
    return MT_OK;
}

uint64_t mt_arena_bytes(const mt_arena *arena) {
    const Arena *a = reinterpret_cast<const Arena *>(arena);
    return a ? a->cursor : 0;
}

int mt_arena_upload(mt_arena *arena, void *device_base, mt_stream_t stream) {
    Arena *a = reinterpret_cast<Arena *>(arena);
    if (!a || (!device_base && a->cursor)) return set_error(MT_EINVAL, "mt_arena_upload: null argument");
    if (a->uploaded) return set_error(MT_EINVAL, "mt_arena_upload: the arena is already uploaded");
    if (reinterpret_cast<uintptr_t>(device_base) % 256)
        return set_error(MT_EINVAL, "mt_arena_upload: the device arena must be 256-byte aligned");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    uint8_t *dev = static_cast<uint8_t *>(device_base);
    constexpr size_t STAGE = size_t(64) << 20;
    uint8_t *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    unsigned long long *counts = nullptr;
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 && e == hipSuccess; i++) e = hipHostMalloc(reinterpret_cast<void **>(&stage[i]), STAGE, 0);
    for (int i = 0; i < 2 && e == hipSuccess; i++) e = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
    if (e == hipSuccess && a->convert_to == MT_F16) e = hipMalloc(&counts, 2 * sizeof(unsigned long long));
    if (e == hipSuccess && counts) e = hipMemsetAsync(counts, 0, 2 * sizeof(unsigned long long), s);
    // Zero the arena first: placement padding and padded columns read as zeros.
    if (e == hipSuccess && a->cursor) e = hipMemsetAsync(dev, 0, a->cursor, s);
    // Host fill of one staging buffer while the other's copy runs.
    int cur = 0;
    size_t used = 0;
    struct Pending {
        uint64_t dst;
        size_t off, bytes;
    };
    std::vector<Pending> pend;
    bool fresh[2] = {true, true};
    auto flush = [&]() {
        for (const Pending &p : pend)
            if (e == hipSuccess) e = hipMemcpyAsync(dev + p.dst, stage[cur] + p.off, p.bytes, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipEventRecord(done[cur], s);
        fresh[cur] = false;
        pend.clear();
        cur ^= 1;
        used = 0;
        if (e == hipSuccess && !fresh[cur]) e = hipEventSynchronize(done[cur]);  // its previous copies are done
    };
    auto put = [&](uint64_t dst, const uint8_t *src, size_t bytes) {
        while (bytes && e == hipSuccess) {
            if (used == STAGE) flush();
            const size_t n = std::min(bytes, STAGE - used);
            memcpy(stage[cur] + used, src, n);
            if (!pend.empty() && pend.back().dst + pend.back().bytes == dst && pend.back().off + pend.back().bytes == used)
                pend.back().bytes += n;
            else
                pend.push_back({dst, used, n});
            used += n;
            dst += n;
            src += n;
            bytes -= n;
        }
    };
    for (const ArenaCopy &c : a->copies) {
        if (e != hipSuccess) break;
        if (c.rows == 0) {
            put(c.dst, c.src, c.bytes);
        } else {
            for (uint32_t r = 0; r < c.rows && e == hipSuccess; r++) put(c.dst + r * c.dst_row, c.src + r * c.src_row, c.src_row);
        }
    }
    if (e == hipSuccess && used) flush();
    if (e == hipSuccess && counts && a->cursor) {
        const uint64_t n8 = a->cursor / 16;  // the arena size is a multiple of 256 bytes
        const unsigned blocks = static_cast<unsigned>(std::min<uint64_t>((n8 + 255) / 256, 4096));
        hipLaunchKernelGGL(bf16_to_f16_kernel, dim3(blocks), dim3(256), 0, s, reinterpret_cast<uint16_t *>(dev), n8,
                           counts);
        e = hipGetLastError();
    }
    unsigned long long host_counts[2] = {0, 0};
    if (e == hipSuccess && counts) e = hipMemcpyAsync(host_counts, counts, sizeof(host_counts), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    for (int i = 0; i < 2; i++) {
        if (done[i]) (void)hipEventDestroy(done[i]);
        if (stage[i]) (void)hipHostFree(stage[i]);
    }
    if (counts) (void)hipFree(counts);
    if (e != hipSuccess) return set_error(MT_EHIP, "mt_arena_upload: %s", hipGetErrorString(e));
    a->overflow = host_counts[0];
    a->underflow = host_counts[1];
    a->uploaded = true;
    return MT_OK;
}

int mt_arena_audit(const mt_arena *arena, uint64_t *overflow, uint64_t *underflow) {
    const Arena *a = reinterpret_cast<const Arena *>(arena);
    if (!a || !overflow || !underflow) return set_error(MT_EINVAL, "mt_arena_audit: null argument");
    if (!a->uploaded) return set_error(MT_EINVAL, "mt_arena_audit: the arena is not uploaded yet");
    *overflow = a->overflow;
    *underflow = a->underflow;
    return MT_OK;
}

int mt_arena_destroy(mt_arena *arena) {
    delete reinterpret_cast<Arena *>(arena);
    return MT_OK;
}

}  // extern "C"
