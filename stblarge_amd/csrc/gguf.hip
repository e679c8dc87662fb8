// GGUF (version 3) reader for expert files: the header is read with pread in growing windows (the
// file is not mapped), the key-value metadata and the tensor table are kept, and tensor offsets are
// made absolute. Only what the expert tier needs is interpreted: scalar and scalar-array values and
// the tensor types of the reference's converted files (stbl/gguf.h:34-36: F32, F16, BF16, I8, MXFP4
// blocks of 17 bytes, and its E4M3 / E8M0 byte tensors). Format: magic "GGUF", version, tensor and
// key counts, keys (string, type, value), tensor infos (name, dims innermost first, type, offset
// relative to the data start), data aligned to general.alignment (32 when absent).
#include <fcntl.h>
#include <unistd.h>

#include <stdint.h>

#include <algorithm>
#include <cstring>

#include <map>
#include <string>
#include <vector>

#include "abi_util.hpp"

namespace stbl {

enum GgufValue : uint32_t { GV_U8, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR, GV_U64, GV_I64, GV_F64 };
enum GgufType : uint32_t { GT_F32 = 0, GT_F16 = 1, GT_I8 = 24, GT_BF16 = 30, GT_MXFP4 = 39, GT_E4M3 = 200, GT_E8M0 = 201 };

struct GgufTensorInfo {
    uint32_t type = 0;
    std::vector<uint64_t> dims;
    uint64_t offset = 0, nbytes = 0;
};

struct GgufFile {
    std::map<std::string, std::pair<uint32_t, std::vector<uint8_t>>> kv;  // type, raw value bytes
    std::map<std::string, GgufTensorInfo> tensors;
    uint64_t size = 0;
};

static uint64_t value_size(uint32_t t) {
    switch (t) {
        case GV_U8: case GV_I8: case GV_BOOL: return 1;
        case GV_U16: case GV_I16: return 2;
        case GV_U32: case GV_I32: case GV_F32: return 4;
        case GV_U64: case GV_I64: case GV_F64: return 8;
        default: return 0;
    }
}

static bool tensor_bytes(uint32_t type, uint64_t n, uint64_t *out) {
    switch (type) {
        case GT_F32: *out = n * 4; return true;
        case GT_F16: case GT_BF16: *out = n * 2; return true;
        case GT_I8: case GT_E4M3: case GT_E8M0: *out = n; return true;
        case GT_MXFP4: *out = n / 32 * 17; return n % 32 == 0;
        default: return false;
    }
}

// Sequential reader over the file's first bytes; refills from the file when the header outgrows the
// window. Throws std::string on malformed input.
struct HeaderReader {
    int fd;
    uint64_t fsize, pos = 0;
    std::vector<uint8_t> buf;
    void need(uint64_t n) {
        if (pos + n <= buf.size()) return;
        if (pos + n > fsize) throw std::string("truncated GGUF header");
        uint64_t want = std::max<uint64_t>(pos + n, std::min<uint64_t>(fsize, std::max<uint64_t>(buf.size() * 2, 1 << 20)));
        const uint64_t have = buf.size();
        buf.resize(want);
        uint64_t got = have;
        while (got < want) {
            const ssize_t r = pread(fd, buf.data() + got, want - got, (off_t)got);
            if (r <= 0) throw std::string("read error in GGUF header");
            got += (uint64_t)r;
        }
    }
    template <class T>
    T get() {
        need(sizeof(T));
        T v;
        memcpy(&v, buf.data() + pos, sizeof(T));
        pos += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (n > (1u << 20)) throw std::string("GGUF string too long");
        need(n);
        std::string s((const char *)buf.data() + pos, n);
        pos += n;
        return s;
    }
    std::vector<uint8_t> value(uint32_t t, int depth = 0) {
        if (depth > 2) throw std::string("GGUF arrays nested too deep");
        if (t == GV_STR) {
            const std::string s = str();
            return std::vector<uint8_t>(s.begin(), s.end());
        }
        if (t == GV_ARR) {
            const uint32_t et = get<uint32_t>();
            const uint64_t n = get<uint64_t>();
            std::vector<uint8_t> out(12);
            memcpy(out.data(), &et, 4);
            memcpy(out.data() + 4, &n, 8);
            if (et == GV_STR || et == GV_ARR) {
                for (uint64_t i = 0; i < n; i++) value(et, depth + 1);  // kept as element type + count only
                return out;
            }
            const uint64_t sz = value_size(et);
            if (!sz || n > (1ull << 32)) throw std::string("bad GGUF array");
            need(n * sz);
            out.insert(out.end(), buf.begin() + pos, buf.begin() + pos + n * sz);
            pos += n * sz;
            return out;
        }
        const uint64_t sz = value_size(t);
        if (!sz) throw std::string("bad GGUF value type");
        need(sz);
        std::vector<uint8_t> out(buf.begin() + pos, buf.begin() + pos + sz);
        pos += sz;
        return out;
    }
};

static GgufFile *parse(const char *path, std::string &err) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        err = std::string("cannot open ") + path;
        return nullptr;
    }
    GgufFile *g = new GgufFile();
    try {
        const off_t end = lseek(fd, 0, SEEK_END);
        if (end < 24) throw std::string("not a GGUF file");
        g->size = (uint64_t)end;
        HeaderReader r{fd, g->size};
        if (r.get<uint32_t>() != 0x46554747u) throw std::string("not a GGUF file");
        if (r.get<uint32_t>() < 2) throw std::string("GGUF version < 2");
        const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
        if (n_tensors > (1u << 24) || n_kv > (1u << 24)) throw std::string("implausible GGUF counts");
        uint64_t alignment = 32;
        for (uint64_t i = 0; i < n_kv; i++) {
            const std::string key = r.str();
            const uint32_t t = r.get<uint32_t>();
            g->kv[key] = {t, r.value(t)};
            if (key == "general.alignment" && t == GV_U32) memcpy(&alignment, g->kv[key].second.data(), 4), alignment &= 0xffffffffu;
        }
        if (!alignment || (alignment & (alignment - 1))) throw std::string("bad general.alignment");
        std::vector<std::pair<std::string, GgufTensorInfo>> list;
        for (uint64_t i = 0; i < n_tensors; i++) {
            std::pair<std::string, GgufTensorInfo> e;
            e.first = r.str();
            const uint32_t nd = r.get<uint32_t>();
            if (nd > 8) throw std::string("tensor with more than 8 dims");
            uint64_t n = 1;
            for (uint32_t d = 0; d < nd; d++) {
                const uint64_t dim = r.get<uint64_t>();
                if (dim && n > (UINT64_MAX >> 5) / dim) throw "tensor " + e.first + " has an implausible shape";
                e.second.dims.push_back(dim);
                n *= dim;
            }
            e.second.type = r.get<uint32_t>();
            e.second.offset = r.get<uint64_t>();
            if (!tensor_bytes(e.second.type, n, &e.second.nbytes)) e.second.nbytes = 0;  // unsupported type
            list.push_back(e);
        }
        const uint64_t data = (r.pos + alignment - 1) / alignment * alignment;
        for (auto &e : list) {
            if (e.second.offset > g->size || data > g->size - e.second.offset ||
                e.second.nbytes > g->size - data - e.second.offset)
                throw "tensor " + e.first + " runs past the end of the file";
            e.second.offset += data;
            g->tensors[e.first] = e.second;
        }
    } catch (const std::string &e) {
        err = e;
        delete g;
        g = nullptr;
    }
    close(fd);
    return g;
}

}  // namespace stbl

using namespace stbl;

extern "C" {

void *stbl_amd_gguf_open(const char *path) {
    if (!path) {
        abi_fail(hipErrorInvalidValue, "gguf_open: null path");
        return nullptr;
    }
    std::string err;
    GgufFile *g = parse(path, err);
    if (!g) abi_fail(hipErrorInvalidValue, "gguf_open: %s", err.c_str());
    return g;
}

void stbl_amd_gguf_close(void *g) { delete (GgufFile *)g; }

int stbl_amd_gguf_tensor(void *g, const char *name, uint32_t *type, uint64_t *dims, int *ndims, uint64_t *offset,
                         uint64_t *nbytes) {
    GgufFile *f = (GgufFile *)g;
    if (!f || !name) return abi_fail(hipErrorInvalidValue, "gguf_tensor: null argument");
    auto it = f->tensors.find(name);
    if (it == f->tensors.end()) return -(int)hipErrorNotFound;  // absent: not recorded as a failure
    const GgufTensorInfo &t = it->second;
    if (type) *type = t.type;
    if (ndims) *ndims = (int)t.dims.size();
    if (dims)
        for (size_t d = 0; d < t.dims.size() && d < 4; d++) dims[d] = t.dims[d];
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return 0;
}

int stbl_amd_gguf_u32(void *g, const char *key, uint32_t *v) {
    GgufFile *f = (GgufFile *)g;
    if (!f || !key || !v) return abi_fail(hipErrorInvalidValue, "gguf_u32: null argument");
    auto it = f->kv.find(key);
    if (it == f->kv.end() || it->second.first != GV_U32) return -(int)hipErrorNotFound;
    memcpy(v, it->second.second.data(), 4);
    return 0;
}

int stbl_amd_gguf_f32(void *g, const char *key, float *v) {
    GgufFile *f = (GgufFile *)g;
    if (!f || !key || !v) return abi_fail(hipErrorInvalidValue, "gguf_f32: null argument");
    auto it = f->kv.find(key);
    if (it == f->kv.end() || it->second.first != GV_F32) return -(int)hipErrorNotFound;
    memcpy(v, it->second.second.data(), 4);
    return 0;
}

// A u32 or u64 array (stbl/gguf.h:31 uints): writes up to cap values into out (may be NULL) and
// returns the array's length, or -hipErrorNotFound when the key is absent or not such an array.
int64_t stbl_amd_gguf_uints(void *g, const char *key, uint64_t *out, int64_t cap) {
    GgufFile *f = (GgufFile *)g;
    if (!f || !key || cap < 0) return abi_fail(hipErrorInvalidValue, "gguf_uints: bad arguments");
    auto it = f->kv.find(key);
    if (it == f->kv.end() || it->second.first != GV_ARR) return -(int)hipErrorNotFound;
    const std::vector<uint8_t> &v = it->second.second;
    uint32_t et;
    uint64_t n;
    memcpy(&et, v.data(), 4);
    memcpy(&n, v.data() + 4, 8);
    if (et != GV_U32 && et != GV_U64) return -(int)hipErrorNotFound;
    for (uint64_t i = 0; out && i < n && (int64_t)i < cap; i++) {
        if (et == GV_U32) {
            uint32_t x;
            memcpy(&x, v.data() + 12 + 4 * i, 4);
            out[i] = x;
        } else {
            memcpy(&out[i], v.data() + 12 + 8 * i, 8);
        }
    }
    return (int64_t)n;
}

}  // extern "C"
