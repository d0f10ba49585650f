/* SPDX-License-Identifier: Unlicense */

/* safetensors reader behind the pth_loader.h API: an 8-byte little-endian
 * header length, a JSON header {name: {dtype, shape, data_offsets}}, the
 * raw tensor data. The JSON subset parsed here is what the format uses:
 * objects, arrays, strings, integers (and __metadata__ skipped). */

#include <ctype.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "common.h"
#include "hip_backend.h"
#include "pth_loader.h"

namespace {

struct parser {
    const char *p, *end;
    const char *path;
    const char *start;

    void fail(const char *what)
    {
        icoreg_fatal("safetensors <%s>: malformed header (%s at byte %ld)",
                     path, what, (long)(p - start));
    }
    void ws()
    {
        while (p < end && isspace((unsigned char)*p))
            p++;
    }
    bool peek(char c)
    {
        ws();
        return p < end && *p == c;
    }
    void expect(char c)
    {
        ws();
        if (p >= end || *p != c)
            fail("unexpected character");
        p++;
    }
    std::string str()
    {
        std::string s;

        expect('"');
        while (p < end && *p != '"') {
            if (*p == '\\') {
                p++;
                if (p >= end)
                    fail("bad escape");
                switch (*p) {
                case 'n':
                    s += '\n';
                    break;
                case 't':
                    s += '\t';
                    break;
                case 'u':
                    /* Tensor names are ASCII; keep the escape text. */
                    s += "\\u";
                    break;
                default:
                    s += *p;
                }
                p++;
                continue;
            }
            s += *p++;
        }
        expect('"');
        return s;
    }
    long long integer()
    {
        long long v = 0;
        int neg = 0;

        ws();
        if (p < end && *p == '-') {
            neg = 1;
            p++;
        }
        if (p >= end || !isdigit((unsigned char)*p))
            fail("number expected");
        while (p < end && isdigit((unsigned char)*p))
            v = v * 10 + (*p++ - '0');
        return neg ? -v : v;
    }
    /* Skip any JSON value. */
    void skip()
    {
        ws();
        if (p >= end)
            fail("value expected");
        if (*p == '"') {
            str();
        }
        else if (*p == '{') {
            p++;
            if (peek('}')) {
                p++;
                return;
            }
            for (;;) {
                str();
                expect(':');
                skip();
                if (peek(',')) {
                    p++;
                    continue;
                }
                expect('}');
                return;
            }
        }
        else if (*p == '[') {
            p++;
            if (peek(']')) {
                p++;
                return;
            }
            for (;;) {
                skip();
                if (peek(',')) {
                    p++;
                    continue;
                }
                expect(']');
                return;
            }
        }
        else {
            while (p < end && *p != ',' && *p != '}' && *p != ']')
                p++;
        }
    }
};

enum pth_dtype parse_dtype(const std::string &s)
{
    if (s == "F32")
        return PTH_F32;
    if (s == "F16")
        return PTH_F16;
    if (s == "BF16")
        return PTH_BF16;
    return PTH_OTHER;
}

size_t dtype_size(const std::string &s)
{
    if (s == "F64" || s == "I64" || s == "U64")
        return 8;
    if (s == "F32" || s == "I32" || s == "U32")
        return 4;
    if (s == "F16" || s == "BF16" || s == "I16" || s == "U16")
        return 2;
    return 1;
}

float half_to_float(uint16_t h)
{
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31,
                   m = h & 1023;
    uint32_t bits;
    float f;

    if (e == 0) {
        f = (float)m * (1.0f / 16777216.0f); /* m * 2^-24 */
        return s ? -f : f;
    }
    if (e == 31)
        bits = s | 0x7f800000u | (m << 13);
    else
        bits = s | ((e + 112) << 23) | (m << 13);
    memcpy(&f, &bits, 4);
    return f;
}

} // namespace

extern "C" void pth_open(struct pth_file *pf, const char *path)
{
    ICOREG_API_BEGIN
    FILE *fp;
    uint64_t hlen = 0;
    std::vector<char> hdr;
    std::vector<struct pth_tensor> ts;
    long long data0, fsize;

    memset(pf, 0, sizeof(*pf));
    if (!(fp = fopen(path, "rb")))
        icoreg_fatal("Unable to open checkpoint <%s>", path);
    fseek(fp, 0, SEEK_END);
    fsize = ftell(fp);
    fseek(fp, 0, SEEK_SET);
    if (fread(&hlen, 8, 1, fp) != 1 || hlen == 0 ||
        (long long)hlen > fsize - 8) {
        fclose(fp);
        icoreg_fatal("Checkpoint <%s> is not a safetensors file (the torch "
                     "zip and pickle formats are not read by this build)",
                     path);
    }
    hdr.resize(hlen);
    if (fread(hdr.data(), 1, hlen, fp) != hlen) {
        fclose(fp);
        icoreg_fatal("Checkpoint <%s>: short header", path);
    }
    data0 = 8 + (long long)hlen;
    {
        parser ps{hdr.data(), hdr.data() + hlen, path, hdr.data()};

        ps.expect('{');
        if (ps.peek('}'))
            ps.p++;
        else
            for (;;) {
                std::string name = ps.str();

                ps.expect(':');
                if (name == "__metadata__") {
                    ps.skip();
                }
                else {
                    struct pth_tensor t;
                    std::string dtype;
                    long long o0 = -1, o1 = -1;
                    size_t esz = 4;

                    memset(&t, 0, sizeof(t));
                    t.ndim = -1;
                    ps.expect('{');
                    for (;;) {
                        std::string key = ps.str();

                        ps.expect(':');
                        if (key == "dtype") {
                            dtype = ps.str();
                        }
                        else if (key == "shape") {
                            ps.expect('[');
                            t.ndim = 0;
                            if (ps.peek(']'))
                                ps.p++;
                            else
                                for (;;) {
                                    long long d = ps.integer();

                                    if (t.ndim >= PTH_MAX_DIMS || d < 0)
                                        ps.fail("shape");
                                    t.shape[t.ndim++] = (long)d;
                                    if (ps.peek(',')) {
                                        ps.p++;
                                        continue;
                                    }
                                    ps.expect(']');
                                    break;
                                }
                        }
                        else if (key == "data_offsets") {
                            ps.expect('[');
                            o0 = ps.integer();
                            ps.expect(',');
                            o1 = ps.integer();
                            ps.expect(']');
                        }
                        else
                            ps.skip();
                        if (ps.peek(',')) {
                            ps.p++;
                            continue;
                        }
                        ps.expect('}');
                        break;
                    }
                    if (t.ndim < 0 || o0 < 0 || o1 < o0 || dtype.empty())
                        icoreg_fatal("Checkpoint <%s>: tensor <%s> lacks "
                                     "dtype, shape or offsets",
                                     path, name.c_str());
                    t.dtype = parse_dtype(dtype);
                    esz = dtype_size(dtype);
                    t.name = strdup(name.c_str());
                    t.data_offset = (long)(data0 + o0);
                    t.storage_bytes = (size_t)(o1 - o0);
                    {
                        long n = 1, s = 1;
                        int d;

                        for (d = 0; d < t.ndim; d++)
                            n *= t.shape[d];
                        for (d = t.ndim - 1; d >= 0; d--) {
                            t.stride[d] = s;
                            s *= t.shape[d];
                        }
                        if ((size_t)n * esz != t.storage_bytes ||
                            data0 + o1 > fsize)
                            icoreg_fatal("Checkpoint <%s>: tensor <%s> size "
                                         "does not match its shape",
                                         path, name.c_str());
                    }
                    ts.push_back(t);
                }
                if (ps.peek(',')) {
                    ps.p++;
                    continue;
                }
                ps.expect('}');
                break;
            }
    }
    pf->fp = fp;
    pf->path = strdup(path);
    pf->ntensors = (int)ts.size();
    pf->tensors = (struct pth_tensor *)calloc(ts.size() + 1, sizeof(ts[0]));
    memcpy(pf->tensors, ts.data(), ts.size() * sizeof(ts[0]));
    ICOREG_API_END
}

extern "C" const struct pth_tensor *pth_find(const struct pth_file *pf,
                                             const char *name)
{
    int i;

    for (i = 0; i < pf->ntensors; i++)
        if (strcmp(pf->tensors[i].name, name) == 0)
            return &pf->tensors[i];
    return NULL;
}

extern "C" const struct pth_tensor *pth_require(const struct pth_file *pf,
                                                const char *name, int ndim,
                                                const long *shape)
{
    const struct pth_tensor *t = NULL;
    ICOREG_API_BEGIN
    int d;

    t = pth_find(pf, name);
    if (!t)
        icoreg_fatal("Checkpoint <%s>: tensor <%s> not found", pf->path, name);
    if (t->dtype == PTH_OTHER)
        icoreg_fatal("Checkpoint <%s>: tensor <%s> is not a float tensor",
                     pf->path, name);
    if (t->ndim != ndim)
        icoreg_fatal("Checkpoint <%s>: tensor <%s> has %d dimensions, %d "
                     "expected",
                     pf->path, name, t->ndim, ndim);
    for (d = 0; d < ndim; d++)
        if (shape[d] >= 0 && shape[d] != t->shape[d])
            icoreg_fatal("Checkpoint <%s>: tensor <%s> dimension %d is %ld, "
                         "%ld expected",
                         pf->path, name, d, t->shape[d], shape[d]);
    ICOREG_API_END_RET(t)
}

extern "C" int pth_strip_prefix(struct pth_file *pf, const char *prefix)
{
    size_t n = strlen(prefix);
    int i, k = 0;

    for (i = 0; i < pf->ntensors; i++)
        if (strncmp(pf->tensors[i].name, prefix, n) == 0) {
            memmove(pf->tensors[i].name, pf->tensors[i].name + n,
                    strlen(pf->tensors[i].name + n) + 1);
            k++;
        }
    return k;
}

extern "C" long pth_numel(const struct pth_tensor *t)
{
    long n = 1;
    int d;

    for (d = 0; d < t->ndim; d++)
        n *= t->shape[d];
    return n;
}

extern "C" double pth_bytes(const struct pth_file *pf, const char *prefix)
{
    size_t n = strlen(prefix);
    double s = 0;
    int i;

    for (i = 0; i < pf->ntensors; i++)
        if (strncmp(pf->tensors[i].name, prefix, n) == 0)
            s += (double)pf->tensors[i].storage_bytes;
    return s;
}

extern "C" float *pth_read_f32(const struct pth_file *pf,
                               const struct pth_tensor *t)
{
    float *out = NULL;
    ICOREG_API_BEGIN
    long n = pth_numel(t), i;
    std::vector<unsigned char> raw(t->storage_bytes);

    if (t->dtype == PTH_OTHER)
        icoreg_fatal("Checkpoint <%s>: tensor <%s> is not a float tensor",
                     pf->path, t->name);
    if (fseek(pf->fp, t->data_offset, SEEK_SET) != 0 ||
        fread(raw.data(), 1, t->storage_bytes, pf->fp) != t->storage_bytes)
        icoreg_fatal("Checkpoint <%s>: reading <%s> failed", pf->path,
                     t->name);
    out = (float *)malloc((n > 0 ? n : 1) * sizeof(float));
    if (t->dtype == PTH_F32)
        memcpy(out, raw.data(), n * sizeof(float));
    else if (t->dtype == PTH_F16)
        for (i = 0; i < n; i++) {
            uint16_t h;

            memcpy(&h, &raw[2 * i], 2);
            out[i] = half_to_float(h);
        }
    else
        for (i = 0; i < n; i++) {
            uint32_t b;

            b = (uint32_t)raw[2 * i] << 16 | (uint32_t)raw[2 * i + 1] << 24;
            memcpy(&out[i], &b, 4);
        }
    ICOREG_API_END_RET(out)
}

extern "C" void pth_close(struct pth_file *pf)
{
    int i;

    if (pf->fp)
        fclose(pf->fp);
    for (i = 0; i < pf->ntensors; i++)
        free(pf->tensors[i].name);
    free(pf->tensors);
    free(pf->path);
    memset(pf, 0, sizeof(*pf));
}
