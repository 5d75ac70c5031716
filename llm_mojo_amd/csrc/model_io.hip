// Saved GPT-2 model files (--save / --weights, gpt2t.mojo:612-698) in
// serialize.mojo's encoding: integers are 8 bytes little-endian, strings a
// length and the bytes, buffers their raw bytes.  The file holds
//   magic, version, W.name(), E.name(),
//   wte (E.save), the 48 layer matrices in load_model's order (W.save),
//   SMALL_FLOATS, the small float32 tensors in Model.small's order,
// where QuantMatrix.save (tensor.mojo:634-644) writes rows, cols, group, the
// codes in the reference's own layout (BLOCKED for int4-g32-a16), the
// float16 scales and the uint8 zero points.  Files written here load in the
// reference and the other way round.
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "gpt2.h"

std::string quant_name(const QFormat &f) {
    std::string s = "int" + std::to_string(f.bits) + "-" + (f.group == 0 ? std::string("ch") : "g" + std::to_string(f.group));
    if (f.sym) s += "-sym";
    return f.a16 ? s + "-a16" : s;
}

bool parse_quant_name(const std::string &s, QFormat *f) {
    for (int b : {4, 8}) {
        const std::string pre = "int" + std::to_string(b) + "-";
        if (s.rfind(pre, 0) != 0) continue;
        int g = 0;
        if (s.compare(pre.size(), 2, "ch") != 0) {
            if (s.size() <= pre.size() + 1 || s[pre.size()] != 'g') continue;
            g = atoi(s.c_str() + pre.size() + 1);
            if (g <= 0) continue;
        }
        for (int sy = 0; sy < 2; sy++)
            for (int a = 0; a < 2; a++) {
                const QFormat q{b, g, sy, a};
                if (quant_name(q) == s) {
                    *f = q;
                    return true;
                }
            }
    }
    return false;
}

namespace {

const char kMagic[] = "llm_mojo GPT-2 124M weights";  // gpt2t.mojo:621
constexpr int64_t kVersion = 1;                        // gpt2t.mojo:622

struct Writer {  // ByteWriter (serialize.mojo:18-57)
    FILE *f = nullptr;
    int64_t written = 0;
    bool ok = true;
    void bytes(const void *p, size_t n) {
        if (ok && n && fwrite(p, 1, n, f) != n) ok = false;
        written += (int64_t)n;
    }
    void i64(int64_t v) {
        uint8_t b[8];
        for (int i = 0; i < 8; i++) b[i] = (uint8_t)((uint64_t)v >> (8 * i));
        bytes(b, 8);
    }
    void str(const std::string &s) {
        i64((int64_t)s.size());
        bytes(s.data(), s.size());
    }
};

struct Reader {  // ByteReader (serialize.mojo:60-114)
    FILE *f = nullptr;
    std::string path;
    int fill(void *p, size_t n) {
        if (n && fread(p, 1, n, f) != n)
            return llmq_set_error(LLMQ_EINVAL, "unexpected end of %s", path.c_str());
        return LLMQ_OK;
    }
    int i64(int64_t *v) {
        uint8_t b[8];
        RC(fill(b, 8));
        uint64_t u = 0;
        for (int i = 0; i < 8; i++) u |= (uint64_t)b[i] << (8 * i);
        *v = (int64_t)u;
        return LLMQ_OK;
    }
    int chars(int64_t n, std::string *s) {
        s->assign((size_t)n, '\0');
        return n ? fill(&(*s)[0], (size_t)n) : LLMQ_OK;
    }
    int str(std::string *s) {
        int64_t n;
        RC(i64(&n));
        if (n < 0 || n > (1 << 20)) return llmq_set_error(LLMQ_EINVAL, "bad string length in %s", path.c_str());
        return chars(n, s);
    }
};

struct FileCloser {
    FILE *f;
    ~FileCloser() {
        if (f) fclose(f);
    }
};

// QuantMatrix.save (tensor.mojo:634-644).
int save_mat(Writer &w, llmq_ctx *ctx, const llmq_mat *m) {
    const int64_t groups = m->n * (m->k / m->group);
    std::vector<uint8_t> codes((size_t)(m->n * m->k * m->bits / 8)), zps((size_t)groups);
    std::vector<uint16_t> scales((size_t)groups);
    RC(llmq_mat_export(ctx, m, codes.data(), scales.data(), zps.data()));
    w.i64(m->n);
    w.i64(m->k);
    w.i64(m->group);
    w.bytes(codes.data(), codes.size());
    w.bytes(scales.data(), scales.size() * 2);
    w.bytes(zps.data(), zps.size());
    return LLMQ_OK;
}

// QuantMatrix.restore (tensor.mojo:646-656) into the device layout; the
// shape must be the one the model expects.
int restore_mat(Reader &r, llmq_ctx *ctx, const QFormat &f, int64_t want_rows, int64_t want_cols, llmq_mat **out) {
    const int bits = f.bits, group = f.group;
    int64_t rows, cols, g;
    RC(r.i64(&rows));
    RC(r.i64(&cols));
    RC(r.i64(&g));
    if (g <= 0 || cols <= 0 || cols % g != 0)
        return llmq_set_error(LLMQ_EINVAL, "bad group size in saved matrix");
    if (rows != want_rows || cols != want_cols || g != (group == 0 ? cols : group))
        return llmq_set_error(LLMQ_EINVAL, "%s: saved matrix %lld x %lld (group %lld), expected %lld x %lld",
                              r.path.c_str(), (long long)rows, (long long)cols, (long long)g,
                              (long long)want_rows, (long long)want_cols);
    const int64_t groups = rows * (cols / g);
    std::vector<uint8_t> codes((size_t)(rows * cols * bits / 8)), zps((size_t)groups);
    std::vector<uint16_t> scales((size_t)groups);
    RC(r.fill(codes.data(), codes.size()));
    RC(r.fill(scales.data(), scales.size() * 2));
    RC(r.fill(zps.data(), zps.size()));
    return llmq_mat_restore(ctx, bits, group, f.sym, f.a16, rows, cols, codes.data(), scales.data(), zps.data(), out);
}

// check_magic (gpt2t.mojo:653-661), then the two format names.
int read_header(Reader &r, std::string *layers, std::string *head) {
    const std::string magic = kMagic;
    int64_t n, version;
    std::string got;
    RC(r.i64(&n));
    if (n != (int64_t)magic.size() || r.chars(n, &got) != LLMQ_OK || got != magic)
        return llmq_set_error(LLMQ_EINVAL, "%s is not a saved llm_mojo model (see --save)", r.path.c_str());
    RC(r.i64(&version));
    if (version != kVersion)
        return llmq_set_error(LLMQ_EINVAL, "%s: unsupported version %lld", r.path.c_str(), (long long)version);
    RC(r.str(layers));
    return r.str(head);
}

}  // namespace

extern "C" {

int llmq_gpt2_save(llmq_gpt2 *m, const char *path) {
    LLMQ_REQUIRE(m && path, "gpt2_save: bad arguments");
    LLMQ_REQUIRE(!m->gguf, "gpt2_save: a model loaded from GGUF keeps its file; save covers QuantMatrix models");
    FILE *f = fopen(path, "wb");
    LLMQ_REQUIRE(f, "gpt2_save: cannot open %s for writing", path);
    FileCloser fc{f};
    Writer w;
    w.f = f;
    const llmq_mat *l0 = m->mats[0];
    w.str(kMagic);
    w.i64(kVersion);
    const llmq_mat *e = m->wte;
    w.str(quant_name(QFormat{l0->bits, l0->group_param, l0->sym, l0->a16}));
    w.str(quant_name(QFormat{e->bits, e->group_param, e->sym, e->a16}));
    RC(save_mat(w, m->ctx, m->wte));
    for (const llmq_mat *q : m->mats) RC(save_mat(w, m->ctx, q));
    std::vector<float> small((size_t)SMALL_FLOATS);
    LLMQ_HIP(hipMemcpyAsync(small.data(), m->small, sizeof(float) * SMALL_FLOATS, hipMemcpyDeviceToHost,
                            m->ctx->stream));
    LLMQ_HIP(hipStreamSynchronize(m->ctx->stream));
    w.i64(SMALL_FLOATS);
    w.bytes(small.data(), small.size() * 4);
    fc.f = nullptr;
    const bool closed = fclose(f) == 0;
    LLMQ_REQUIRE(w.ok && closed, "gpt2_save: writing %s failed", path);
    return LLMQ_OK;
}

int llmq_saved_formats(const char *path, char *layers, char *head, int cap) {
    LLMQ_REQUIRE(path && layers && head && cap > 0, "saved_formats: bad arguments");
    FILE *f = fopen(path, "rb");
    LLMQ_REQUIRE(f, "cannot open %s", path);
    FileCloser fc{f};
    Reader r;
    r.f = f;
    r.path = path;
    std::string l, h;
    RC(read_header(r, &l, &h));
    LLMQ_REQUIRE((int)l.size() < cap && (int)h.size() < cap, "saved_formats: names longer than %d", cap - 1);
    memcpy(layers, l.c_str(), l.size() + 1);
    memcpy(head, h.c_str(), h.size() + 1);
    return LLMQ_OK;
}

int llmq_gpt2_load(llmq_ctx *ctx, const char *path, int attention, llmq_gpt2 **out) {
    LLMQ_REQUIRE(ctx && path && out, "gpt2_load: bad arguments");
    LLMQ_REQUIRE(attention == LLMQ_ATTN_FLOAT || attention == LLMQ_ATTN_INT, "gpt2_load: attention %d", attention);
    FILE *f = fopen(path, "rb");
    LLMQ_REQUIRE(f, "cannot open %s", path);
    FileCloser fc{f};
    Reader r;
    r.f = f;
    r.path = path;
    std::string layers, head;
    RC(read_header(r, &layers, &head));
    // main's --weights (gpt2t.mojo:1298-1303): the head is "same" when both
    // names agree, else int8 per channel (HEAD8 or HEAD8_A16 as W is A16)
    QFormat fw, fe;
    const bool ok = parse_quant_name(layers, &fw) && parse_quant_name(head, &fe) &&
                    (fe == fw || fe == QFormat{8, 0, 0, fw.a16});
    if (!ok)
        return llmq_set_error(LLMQ_EUNSUPPORTED, "%s holds %s + head %s; the device model runs QuantMatrix layers "
                              "with head int8-ch (-a16 as the layers) or the layers' own format", path,
                              layers.c_str(), head.c_str());
    llmq_gpt2 *m = new llmq_gpt2();
    m->ctx = ctx;
    int rc = restore_mat(r, ctx, fe, V, C, &m->wte);
    static const int64_t rows[4] = {3 * C, C, 4 * C, C}, cols[4] = {C, C, C, 4 * C};  // [OUT, IN]
    for (int i = 0; rc == LLMQ_OK && i < NL * 4; i++)
        rc = restore_mat(r, ctx, fw, rows[i % 4], cols[i % 4], &m->mats[i]);
    std::vector<float> small;
    if (rc == LLMQ_OK) {
        int64_t n = 0;
        rc = r.i64(&n);
        if (rc == LLMQ_OK && n != SMALL_FLOATS)
            rc = llmq_set_error(LLMQ_EINVAL, "%s: unexpected size of the float32 tensors", path);
    }
    if (rc == LLMQ_OK) {
        small.resize((size_t)SMALL_FLOATS);
        rc = r.fill(small.data(), small.size() * 4);
    }
    if (rc == LLMQ_OK) rc = gpt2_finish(m, attention, small.data());
    if (rc != LLMQ_OK) {
        llmq_gpt2_free(m);
        return rc;
    }
    *out = m;
    return LLMQ_OK;
}

}  // extern "C"
