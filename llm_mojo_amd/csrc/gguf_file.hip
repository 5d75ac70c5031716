// GGUFFile (gguf.mojo:519-636): a GGUF v2 / v3 file's tensor index, with
// the tensors' bytes read in place from a read-only mapping of the file.
//
// Layout (the reference's reader, gguf.mojo:553-590): "GGUF", u32 version
// (>= 2), u64 tensor count, u64 metadata count; metadata entries (string
// key, u32 type, value; only general.alignment is used, default 32); tensor
// infos (string name, u32 dims, u64 dims[], u32 ggml type, u64 offset from
// the data section); the data section starts at the next multiple of the
// alignment.  Strings are a u64 length and the bytes; everything is little-
// endian.  Unlike the reference, every read is bounds-checked, so a
// truncated or corrupt file is an error, not an out-of-range read.
#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"

struct llmq_gguf {
    const uint8_t *buf = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    int64_t data_start = 0;
    int64_t alignment = 32;
    struct Info {
        std::string name;
        int type;
        int64_t cols, rows, offset;  // TensorInfo (gguf.mojo:519-524)
    };
    std::vector<Info> tensors;
    std::unordered_map<std::string, int64_t> index;
};

namespace {

struct Cursor {
    const uint8_t *p;
    size_t size, pos;
    bool ok = true;
    bool need(size_t n) {
        if (!ok || n > size || pos > size - n) ok = false;
        return ok;
    }
    void advance(size_t n) {
        if (need(n)) pos += n;
    }
    uint64_t uint(int bytes) {
        if (!need((size_t)bytes)) return 0;
        uint64_t v = 0;
        for (int i = 0; i < bytes; i++) v |= (uint64_t)p[pos + i] << (8 * i);
        pos += (size_t)bytes;
        return v;
    }
    std::string str() {
        const uint64_t n = uint(8);
        if (!need((size_t)n)) return std::string();
        std::string s(reinterpret_cast<const char *>(p + pos), (size_t)n);
        pos += (size_t)n;
        return s;
    }
    // skip_value (gguf.mojo:600-620) for metadata type t; depth bounds
    // nested arrays.
    void skip(uint32_t t, int depth = 0) {
        switch (t) {
        case 0: case 1: case 7: advance(1); return;     // u8, i8, bool
        case 2: case 3: advance(2); return;             // u16, i16
        case 4: case 5: case 6: advance(4); return;     // u32, i32, f32
        case 10: case 11: case 12: advance(8); return;  // u64, i64, f64
        case 8: (void)str(); return;                    // string
        case 9: {                                                // array
            const uint32_t et = (uint32_t)uint(4);
            const uint64_t count = uint(8);
            if (depth > 8) {
                ok = false;
                return;
            }
            for (uint64_t i = 0; ok && i < count; i++) skip(et, depth + 1);
            return;
        }
        default: ok = false;  // the reference aborts on an unknown type
        }
    }
};

int parse(llmq_gguf *g, const char *path) {
    Cursor c{g->buf, g->size, 0};
    if (c.uint(4) != 0x46554747u || !c.ok)  // "GGUF"
        return llmq_set_error(LLMQ_EINVAL, "%s is not a GGUF file", path);
    g->version = (uint32_t)c.uint(4);
    if (g->version < 2) return llmq_set_error(LLMQ_EUNSUPPORTED, "GGUF version %u is not supported", g->version);
    const uint64_t n_tensors = c.uint(8), n_kv = c.uint(8);
    for (uint64_t i = 0; c.ok && i < n_kv; i++) {
        const std::string key = c.str();
        const uint32_t t = (uint32_t)c.uint(4);
        if (key == "general.alignment" && t == 4) {
            const size_t at = c.pos;
            g->alignment = (int64_t)c.uint(4);
            c.pos = at;
        }
        c.skip(t);
    }
    if (!c.ok) return llmq_set_error(LLMQ_EINVAL, "%s: corrupt or truncated GGUF metadata", path);
    if (g->alignment <= 0) return llmq_set_error(LLMQ_EINVAL, "%s: bad general.alignment", path);
    for (uint64_t i = 0; c.ok && i < n_tensors; i++) {
        llmq_gguf::Info t;
        t.name = c.str();
        const uint32_t ndims = (uint32_t)c.uint(4);
        if (!c.ok || ndims < 1 || ndims > 8) return llmq_set_error(LLMQ_EINVAL, "%s: bad tensor dims", path);
        t.cols = (int64_t)c.uint(8);
        t.rows = 1;
        for (uint32_t d = 1; d < ndims; d++) {
            const uint64_t dim = c.uint(8);
            int64_t r = 0;  // 0 marks an impossible shape (refused below)
            if (t.rows > 0 && dim > 0 && dim <= ((uint64_t)1 << 40) && !__builtin_mul_overflow(t.rows, (int64_t)dim, &r) &&
                r <= ((int64_t)1 << 40))
                t.rows = r;
            else
                t.rows = 0;
        }
        t.type = (int)c.uint(4);
        t.offset = (int64_t)c.uint(8);
        if (!c.ok) break;
        if (t.cols <= 0 || t.rows <= 0 || t.cols > ((int64_t)1 << 40) / t.rows)
            return llmq_set_error(LLMQ_EINVAL, "%s: tensor %s has an impossible shape", path, t.name.c_str());
        g->index[t.name] = (int64_t)g->tensors.size();
        g->tensors.push_back(std::move(t));
    }
    if (!c.ok) return llmq_set_error(LLMQ_EINVAL, "%s: corrupt or truncated GGUF tensor index", path);
    g->data_start = ((int64_t)c.pos + g->alignment - 1) / g->alignment * g->alignment;
    return LLMQ_OK;
}

// Bytes of a tensor (gguf.mojo:72-98); 0 for a type without a block size.
int64_t tensor_bytes(const llmq_gguf::Info &t) {
    const int bs = t.type == LLMQ_GGML_F32 || t.type == LLMQ_GGML_F16 ? 1 : gguf_block_size(t.type);
    const int bb = t.type == LLMQ_GGML_F32 ? 4 : t.type == LLMQ_GGML_F16 ? 2 : gguf_block_bytes(t.type);
    if (bs == 0 || t.cols % bs != 0) return 0;
    return t.rows * (t.cols / bs) * bb;
}

}  // namespace

extern "C" {

int llmq_gguf_open(const char *path, llmq_gguf **out) {
    LLMQ_REQUIRE(path && out, "gguf_open: bad arguments");
    const int fd = open(path, O_RDONLY);
    LLMQ_REQUIRE(fd >= 0, "cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return llmq_set_error(LLMQ_EINVAL, "%s is not a GGUF file", path);
    }
    void *p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    LLMQ_REQUIRE(p != MAP_FAILED, "cannot map %s", path);
    llmq_gguf *g = new llmq_gguf();
    g->buf = static_cast<const uint8_t *>(p);
    g->size = (size_t)st.st_size;
    const int rc = parse(g, path);
    if (rc != LLMQ_OK) {
        llmq_gguf_close(g);
        return rc;
    }
    *out = g;
    return LLMQ_OK;
}

int llmq_gguf_close(llmq_gguf *g) {
    if (!g) return LLMQ_OK;
    if (g->buf) munmap(const_cast<uint8_t *>(g->buf), g->size);
    delete g;
    return LLMQ_OK;
}

int64_t llmq_gguf_n_tensors(const llmq_gguf *g) { return g ? (int64_t)g->tensors.size() : 0; }

int llmq_gguf_find(const llmq_gguf *g, const char *name, int64_t *index) {
    LLMQ_REQUIRE(g && name && index, "gguf_find: bad arguments");
    auto it = g->index.find(name);
    *index = it == g->index.end() ? -1 : it->second;
    return LLMQ_OK;
}

int llmq_gguf_tensor_info(const llmq_gguf *g, int64_t i, const char **name, int *type, int64_t *rows, int64_t *cols,
                          int64_t *offset) {
    LLMQ_REQUIRE(g && i >= 0 && i < (int64_t)g->tensors.size(), "gguf_tensor_info: index out of range");
    const auto &t = g->tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    if (type) *type = t.type;
    if (rows) *rows = t.rows;
    if (cols) *cols = t.cols;
    if (offset) *offset = t.offset;
    return LLMQ_OK;
}

int llmq_gguf_tensor_data(const llmq_gguf *g, int64_t i, const void **data, int64_t *bytes) {
    LLMQ_REQUIRE(g && data && i >= 0 && i < (int64_t)g->tensors.size(), "gguf_tensor_data: bad arguments");
    const auto &t = g->tensors[(size_t)i];
    const int64_t n = tensor_bytes(t);
    LLMQ_REQUIRE(n > 0, "%s: unsupported format (ggml type %d)", t.name.c_str(), t.type);
    // unsigned comparisons with no sum that can wrap
    const uint64_t size = g->size, start = (uint64_t)g->data_start, off = (uint64_t)t.offset, len = (uint64_t)n;
    LLMQ_REQUIRE(t.offset >= 0 && start <= size && len <= size - start && off <= size - start - len,
                 "%s: tensor data past the end of the file", t.name.c_str());
    *data = g->buf + g->data_start + t.offset;
    if (bytes) *bytes = n;
    return LLMQ_OK;
}

int llmq_gguf_matrix(llmq_ctx *ctx, const llmq_gguf *g, const char *name, llmq_mat **out) {
    LLMQ_REQUIRE(ctx && g && name && out, "gguf_matrix: bad arguments");
    auto it = g->index.find(name);
    LLMQ_REQUIRE(it != g->index.end(), "tensor not in GGUF file: %s", name);
    const auto &t = g->tensors[(size_t)it->second];
    const void *data;
    RC(llmq_gguf_tensor_data(g, it->second, &data, nullptr));
    return llmq_mat_from_gguf(ctx, t.type, data, t.rows, t.cols, out);
}

}  // extern "C"
