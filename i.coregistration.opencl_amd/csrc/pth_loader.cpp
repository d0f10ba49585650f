/* SPDX-License-Identifier: Unlicense */

/* Checkpoint reader behind the pth_loader.h API of the reference
 * (pth_loader.h:9-61 of i.coregistration.opencl). It reads the three
 * formats the reference's pth_loader.c reads, told apart by their first
 * bytes:
 *
 *  - safetensors (pth_loader.c:1014-1146): an 8-byte little-endian header
 *    length, a JSON header {name: {dtype, shape, data_offsets}}, the raw
 *    tensor data;
 *  - torch.save's zip archive (pth_loader.c:816-868): <root>/data.pkl
 *    holds the pickled object, <root>/data/<key> each storage, as stored
 *    (uncompressed) entries, Zip64 records included;
 *  - torch.save's legacy stream (pth_loader.c:870-933): five pickles
 *    (magic number, protocol version 1001, system information, the
 *    object, the list of storage keys), then each storage in the order of
 *    that list as an int64 element count and the raw elements.
 *
 * Pickles run on a small stack machine that only builds plain values:
 * module globals are kept as names and are never resolved or called.
 * REDUCE builds tensors from torch's rebuild functions (_rebuild_tensor,
 * _rebuild_tensor_v2/v3, _rebuild_parameter[_with_state],
 * _rebuild_from_type_v2) and dictionaries from collections.OrderedDict;
 * any other call yields an opaque value. The state_dict is the root
 * dictionary if it holds tensors, else its "model" or "state_dict"
 * entry, else its only entry that is a dictionary of tensors ("extractor"
 * in DISK's checkpoints), as pth_loader.c:693-740 chooses it.
 *
 * Tensors of float32, float16 and bfloat16 storages are indexed, with
 * their strides and storage offsets (shared storages and transposed
 * views read correctly); integer and boolean tensors (BatchNorm's
 * num_batches_tracked) are left out, in every format. Every format or
 * lookup problem is a fatal error naming the file. */

#include <ctype.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "hip_backend.h"
#include "pth_loader.h"

namespace {

/* ---- file access ------------------------------------------------------------ */

struct file_ref {
    FILE *fp = nullptr;
    std::string path;
    long long size = 0;

    ~file_ref()
    {
        if (fp)
            fclose(fp);
    }
    void read_at(long long off, void *dst, size_t n) const
    {
        if (off < 0 || off + (long long)n > size ||
            fseeko(fp, (off_t)off, SEEK_SET) != 0 ||
            (n && fread(dst, 1, n, fp) != n))
            icoreg_fatal("Checkpoint <%s>: read of %zu bytes at %lld failed "
                         "(file of %lld bytes)",
                         path.c_str(), n, off, size);
    }
    std::vector<unsigned char> bytes(long long off, size_t n) const
    {
        std::vector<unsigned char> v(n);
        read_at(off, v.data(), n);
        return v;
    }
};

uint64_t le(const unsigned char *p, int n)
{
    uint64_t v = 0;

    for (int k = n - 1; k >= 0; k--)
        v = v << 8 | p[k];
    return v;
}

size_t elem_bytes(enum pth_dtype d) { return d == PTH_F32 ? 4 : 2; }

/* ---- safetensors JSON header ------------------------------------------------ */

struct json_parser {
    const char *p, *end;
    const char *path;
    const char *start;

    [[noreturn]] void fail(const char *what)
    {
        icoreg_fatal("safetensors <%s>: malformed header (%s at byte %ld)",
                     path, what, (long)(p - start));
        abort();
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
        else if (*p == '{' || *p == '[') {
            const char close = *p == '{' ? '}' : ']';
            const bool obj = *p == '{';

            p++;
            if (peek(close)) {
                p++;
                return;
            }
            for (;;) {
                if (obj) {
                    str();
                    expect(':');
                }
                skip();
                if (peek(',')) {
                    p++;
                    continue;
                }
                expect(close);
                return;
            }
        }
        else {
            while (p < end && *p != ',' && *p != '}' && *p != ']')
                p++;
        }
    }
};

/* Element size of a safetensors dtype name and the dtype it maps to. */
size_t st_dtype(const std::string &s, enum pth_dtype *d)
{
    *d = s == "F32" ? PTH_F32 : s == "F16" ? PTH_F16 : s == "BF16" ? PTH_BF16 : PTH_OTHER;
    if (s == "F64" || s == "I64" || s == "U64")
        return 8;
    if (s == "F32" || s == "I32" || s == "U32")
        return 4;
    if (s == "F16" || s == "BF16" || s == "I16" || s == "U16")
        return 2;
    return 1;
}

void contiguous_strides(struct pth_tensor *t)
{
    long s = 1;

    for (int d = t->ndim - 1; d >= 0; d--) {
        t->stride[d] = s;
        s *= t->shape[d];
    }
}

void open_safetensors(const file_ref &f, std::vector<struct pth_tensor> &ts)
{
    const char *path = f.path.c_str();
    unsigned char h8[8];
    uint64_t hlen;
    long long data0;

    f.read_at(0, h8, 8);
    hlen = le(h8, 8);
    if (hlen == 0 || (long long)hlen > f.size - 8)
        icoreg_fatal("Checkpoint <%s> is neither a zip archive, a legacy "
                     "pickle nor a safetensors file",
                     path);
    std::vector<unsigned char> hdr = f.bytes(8, hlen);
    data0 = 8 + (long long)hlen;
    json_parser ps{(const char *)hdr.data(), (const char *)hdr.data() + hlen, path,
                   (const char *)hdr.data()};

    ps.expect('{');
    if (ps.peek('}')) {
        ps.p++;
        return;
    }
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
                icoreg_fatal("Checkpoint <%s>: tensor <%s> lacks dtype, shape or "
                             "offsets",
                             path, name.c_str());
            const size_t esz = st_dtype(dtype, &t.dtype);
            long long n = 1, nb = 0;
            bool wrap = false;

            for (int d = 0; d < t.ndim; d++)
                wrap |= __builtin_mul_overflow(n, (long long)t.shape[d], &n);
            wrap |= __builtin_mul_overflow(n, (long long)esz, &nb);
            if (wrap || nb != o1 - o0 || data0 + o1 > f.size)
                icoreg_fatal("Checkpoint <%s>: tensor <%s> size does not match "
                             "its shape",
                             path, name.c_str());
            /* Integer and boolean tensors are not part of the index. */
            if (t.dtype != PTH_OTHER) {
                t.name = strdup(name.c_str());
                t.data_offset = (long)(data0 + o0);
                t.storage_bytes = (size_t)(o1 - o0);
                contiguous_strides(&t);
                ts.push_back(t);
            }
        }
        if (ps.peek(',')) {
            ps.p++;
            continue;
        }
        ps.expect('}');
        break;
    }
}

/* ---- zip archive ------------------------------------------------------------ */

struct zip_entry {
    std::string name;
    long long data; /* byte offset of the stored data */
    long long size;
};

/* The central directory of a zip archive (EOCD, optionally Zip64), with
 * every entry's data offset resolved through its local header. Entries
 * must be stored: torch.save writes them uncompressed. */
std::vector<zip_entry> zip_entries(const file_ref &f)
{
    const char *path = f.path.c_str();
    const long long tail = f.size < 65557 ? f.size : 65557;
    std::vector<unsigned char> t = f.bytes(f.size - tail, tail);
    long long eocd = -1;
    uint64_t nent, cd_size, cd_off;

    for (long long k = tail - 22; k >= 0; k--)
        if (le(&t[k], 4) == 0x06054b50u) {
            eocd = k;
            break;
        }
    if (eocd < 0)
        icoreg_fatal("Checkpoint <%s>: zip end-of-directory record not found", path);
    nent = le(&t[eocd + 10], 2);
    cd_size = le(&t[eocd + 12], 4);
    cd_off = le(&t[eocd + 16], 4);
    if (nent == 0xffff || cd_size == 0xffffffffu || cd_off == 0xffffffffu) {
        /* Zip64: a 20-byte locator right before the record points at the
         * Zip64 end-of-directory record. */
        if (eocd < 20 || le(&t[eocd - 20], 4) != 0x07064b50u)
            icoreg_fatal("Checkpoint <%s>: Zip64 locator missing", path);
        const long long z64 = (long long)le(&t[eocd - 20 + 8], 8);
        std::vector<unsigned char> r = f.bytes(z64, 56);

        if (le(&r[0], 4) != 0x06064b50u)
            icoreg_fatal("Checkpoint <%s>: bad Zip64 end-of-directory record", path);
        nent = le(&r[32], 8);
        cd_size = le(&r[40], 8);
        cd_off = le(&r[48], 8);
    }
    std::vector<unsigned char> cd = f.bytes((long long)cd_off, cd_size);
    std::vector<zip_entry> out;
    size_t p = 0;

    for (uint64_t e = 0; e < nent; e++) {
        if (p + 46 > cd.size() || le(&cd[p], 4) != 0x02014b50u)
            icoreg_fatal("Checkpoint <%s>: bad zip central directory", path);
        const unsigned method = (unsigned)le(&cd[p + 10], 2);
        uint64_t csize = le(&cd[p + 20], 4), usize = le(&cd[p + 24], 4);
        const size_t nlen = le(&cd[p + 28], 2), xlen = le(&cd[p + 30], 2),
                     clen = le(&cd[p + 32], 2);
        uint64_t loff = le(&cd[p + 42], 4);

        if (p + 46 + nlen + xlen + clen > cd.size())
            icoreg_fatal("Checkpoint <%s>: bad zip central directory", path);
        zip_entry z;
        z.name.assign((const char *)&cd[p + 46], nlen);
        /* Zip64 extra field: the 64-bit sizes and offset, each present
         * only where the 32-bit field is saturated, in this order. */
        for (size_t x = p + 46 + nlen; x + 4 <= p + 46 + nlen + xlen;) {
            const unsigned id = (unsigned)le(&cd[x], 2), sz = (unsigned)le(&cd[x + 2], 2);
            size_t q = x + 4;

            if (id == 1) {
                if (usize == 0xffffffffu && q + 8 <= x + 4 + sz) {
                    usize = le(&cd[q], 8);
                    q += 8;
                }
                if (csize == 0xffffffffu && q + 8 <= x + 4 + sz) {
                    csize = le(&cd[q], 8);
                    q += 8;
                }
                if (loff == 0xffffffffu && q + 8 <= x + 4 + sz)
                    loff = le(&cd[q], 8);
            }
            x += 4 + sz;
        }
        if (method != 0 || csize != usize)
            icoreg_fatal("Checkpoint <%s>: zip entry <%s> is compressed (method "
                         "%u); torch.save writes stored entries",
                         path, z.name.c_str(), method);
        unsigned char lh[30];
        f.read_at((long long)loff, lh, 30);
        if (le(lh, 4) != 0x04034b50u)
            icoreg_fatal("Checkpoint <%s>: bad zip local header of <%s>", path,
                         z.name.c_str());
        z.data = (long long)loff + 30 + (long long)le(lh + 26, 2) + (long long)le(lh + 28, 2);
        z.size = (long long)usize;
        if (z.data + z.size > f.size)
            icoreg_fatal("Checkpoint <%s>: zip entry <%s> runs past the end", path,
                         z.name.c_str());
        out.push_back(std::move(z));
        p += 46 + nlen + xlen + clen;
    }
    return out;
}

/* ---- pickle values and machine ---------------------------------------------- */

enum kind {
    K_NONE, K_BOOL, K_INT, K_BIGINT, K_FLOAT, K_STR, K_TUPLE, K_LIST, K_DICT,
    K_SET, K_GLOBAL, K_STORAGE, K_TENSOR, K_OBJECT
};

struct value;
using val = std::shared_ptr<value>;

struct value {
    kind k = K_NONE;
    long long i = 0;         /* int, bool; storage: element offset of a view */
    double f = 0;
    std::string s, s2;       /* str / bytes; global: module, name; storage: key;
                                bigint: little-endian two's-complement bytes */
    std::vector<val> items;  /* tuple, list, set; dict: key, value, key, ... */
    /* storage */
    enum pth_dtype dtype = PTH_OTHER;
    int elsize = 0;
    /* tensor */
    val storage;
    long long offset = 0;
    std::vector<long long> shape, stride;
};

val mk(kind k)
{
    val v = std::make_shared<value>();
    v->k = k;
    return v;
}

struct unpickler {
    const unsigned char *p, *end, *base;
    const char *path;
    std::vector<val> stack;
    std::vector<size_t> marks;
    std::unordered_map<long long, val> memo;
    std::vector<val> storages; /* every storage value met, for the legacy sizes */

    unpickler(const std::vector<unsigned char> &buf, const char *file)
        : p(buf.data()), end(buf.data() + buf.size()), base(buf.data()), path(file)
    {
    }

    [[noreturn]] void fail(const char *what)
    {
        icoreg_fatal("Checkpoint <%s>: %s in pickle", path, what);
        abort();
    }
    const unsigned char *take(size_t n)
    {
        if ((size_t)(end - p) < n)
            fail("truncated data");
        const unsigned char *q = p;
        p += n;
        return q;
    }
    uint64_t u(int n) { return le(take(n), n); }
    std::string line()
    {
        const unsigned char *q = p;

        while (q < end && *q != '\n')
            q++;
        if (q >= end)
            fail("unterminated line");
        std::string s((const char *)p, q - p);
        p = q + 1;
        return s;
    }
    void push(val v) { stack.push_back(std::move(v)); }
    val pop()
    {
        if (stack.empty() || (!marks.empty() && stack.size() <= marks.back()))
            fail("stack underflow");
        val v = stack.back();
        stack.pop_back();
        return v;
    }
    val &top()
    {
        if (stack.empty() || (!marks.empty() && stack.size() <= marks.back()))
            fail("stack underflow");
        return stack.back();
    }
    /* The values above the last mark, removed with the mark. */
    std::vector<val> pop_mark()
    {
        if (marks.empty())
            fail("missing mark");
        const size_t m = marks.back();
        marks.pop_back();
        std::vector<val> v(stack.begin() + m, stack.end());
        stack.resize(m);
        return v;
    }
    val str(const unsigned char *s, size_t n)
    {
        val v = mk(K_STR);
        v->s.assign((const char *)s, n);
        return v;
    }
    val integer(long long x)
    {
        val v = mk(K_INT);
        v->i = x;
        return v;
    }
    /* Two's-complement little-endian integer of n bytes (LONG1 / LONG4);
     * wider than 64 bits (the legacy format's magic number) it is kept
     * as its bytes. */
    val long_bytes(size_t n)
    {
        const unsigned char *b = take(n);
        long long x = 0;

        if (n > 8) {
            val v = mk(K_BIGINT);
            v->s.assign((const char *)b, n);
            return v;
        }
        for (size_t k = 0; k < n; k++)
            x |= (long long)((uint64_t)b[k] << (8 * k));
        if (n && n < 8 && (b[n - 1] & 0x80))
            x -= (long long)((uint64_t)1 << (8 * n));
        return integer(x);
    }
    val tuple(std::vector<val> items)
    {
        val v = mk(K_TUPLE);
        v->items = std::move(items);
        return v;
    }
    static long long as_int(const val &v, unpickler *m)
    {
        if (v->k != K_INT && v->k != K_BOOL)
            m->fail("integer expected");
        return v->i;
    }
    static bool is_global(const val &v, const char *mod, const char *name)
    {
        return v->k == K_GLOBAL && v->s == mod && v->s2 == name;
    }

    /* A persistent id: ('storage', <module>.<Type>Storage, key, location,
     * numel[, view metadata]). */
    val persistent(const val &pid)
    {
        if (pid->k != K_TUPLE || pid->items.size() < 5 || pid->items[0]->k != K_STR ||
            pid->items[0]->s != "storage" || pid->items[1]->k != K_GLOBAL ||
            pid->items[2]->k != K_STR)
            fail("unsupported persistent id (not a tensor storage)");
        static const std::map<std::string, std::pair<enum pth_dtype, int>> types = {
            {"FloatStorage", {PTH_F32, 4}},   {"HalfStorage", {PTH_F16, 2}},
            {"BFloat16Storage", {PTH_BF16, 2}}, {"DoubleStorage", {PTH_OTHER, 8}},
            {"LongStorage", {PTH_OTHER, 8}},  {"IntStorage", {PTH_OTHER, 4}},
            {"ShortStorage", {PTH_OTHER, 2}}, {"CharStorage", {PTH_OTHER, 1}},
            {"ByteStorage", {PTH_OTHER, 1}},  {"BoolStorage", {PTH_OTHER, 1}},
            {"UntypedStorage", {PTH_OTHER, 1}}};
        auto it = types.find(pid->items[1]->s2);

        if (it == types.end())
            icoreg_fatal("Checkpoint <%s>: unsupported storage type <%s.%s>", path,
                         pid->items[1]->s.c_str(), pid->items[1]->s2.c_str());
        val v = mk(K_STORAGE);
        v->dtype = it->second.first;
        v->elsize = it->second.second;
        v->s = pid->items[2]->s;
        /* Legacy view metadata (view key, element offset, size). */
        if (pid->items.size() >= 6 && pid->items[5]->k == K_TUPLE &&
            pid->items[5]->items.size() >= 2)
            v->i = as_int(pid->items[5]->items[1], this);
        storages.push_back(v);
        return v;
    }

    val reduce(const val &fn, const val &args)
    {
        if (args->k != K_TUPLE)
            fail("REDUCE without an argument tuple");
        const std::vector<val> &a = args->items;

        if (is_global(fn, "torch._utils", "_rebuild_tensor") ||
            is_global(fn, "torch._utils", "_rebuild_tensor_v2") ||
            is_global(fn, "torch._utils", "_rebuild_tensor_v3")) {
            if (a.size() < 4 || a[0]->k != K_STORAGE || a[2]->k != K_TUPLE ||
                a[3]->k != K_TUPLE || a[2]->items.size() != a[3]->items.size())
                fail("unexpected tensor rebuild arguments");
            if (a[2]->items.size() > PTH_MAX_DIMS)
                icoreg_fatal("Checkpoint <%s>: tensor of rank %zu (at most %d)", path,
                             a[2]->items.size(), PTH_MAX_DIMS);
            val t = mk(K_TENSOR);
            t->storage = a[0];
            t->offset = as_int(a[1], this) + a[0]->i;
            for (size_t d = 0; d < a[2]->items.size(); d++) {
                t->shape.push_back(as_int(a[2]->items[d], this));
                t->stride.push_back(as_int(a[3]->items[d], this));
            }
            /* v3 carries its dtype apart from an untyped storage: the
             * dtypes it is used for are not float32 / float16 / bfloat16. */
            if (is_global(fn, "torch._utils", "_rebuild_tensor_v3")) {
                val s = mk(K_STORAGE);
                *s = *a[0];
                s->dtype = PTH_OTHER;
                t->storage = s;
            }
            return t;
        }
        if (is_global(fn, "torch._utils", "_rebuild_parameter") ||
            is_global(fn, "torch._utils", "_rebuild_parameter_with_state")) {
            if (a.empty() || a[0]->k != K_TENSOR)
                fail("unexpected parameter rebuild arguments");
            return a[0];
        }
        /* A tensor subclass: (rebuild function, type, its arguments, state). */
        if (is_global(fn, "torch._tensor", "_rebuild_from_type_v2")) {
            if (a.size() < 3 || a[0]->k != K_GLOBAL || a[2]->k != K_TUPLE)
                fail("unexpected tensor subclass rebuild arguments");
            return reduce(a[0], a[2]);
        }
        if (is_global(fn, "collections", "OrderedDict") ||
            is_global(fn, "builtins", "dict") || is_global(fn, "__builtin__", "dict")) {
            val d = mk(K_DICT);
            /* OrderedDict([(k, v), ...]) */
            if (!a.empty() && a[0]->k == K_LIST)
                for (const val &kv : a[0]->items)
                    if ((kv->k == K_TUPLE || kv->k == K_LIST) && kv->items.size() == 2) {
                        d->items.push_back(kv->items[0]);
                        d->items.push_back(kv->items[1]);
                    }
            return d;
        }
        return mk(K_OBJECT);
    }

    void set_items(val &d, const std::vector<val> &kv)
    {
        if (kv.size() % 2)
            fail("odd SETITEMS");
        if (d->k != K_DICT)
            return; /* items of an opaque object: dropped */
        for (size_t k = 0; k < kv.size(); k += 2) {
            bool done = false;

            /* A repeated string key replaces the earlier value. */
            if (kv[k]->k == K_STR)
                for (size_t q = 0; q < d->items.size(); q += 2)
                    if (d->items[q]->k == K_STR && d->items[q]->s == kv[k]->s) {
                        d->items[q + 1] = kv[k + 1];
                        done = true;
                        break;
                    }
            if (!done) {
                d->items.push_back(kv[k]);
                d->items.push_back(kv[k + 1]);
            }
        }
    }

    /* Runs one pickle to its STOP and returns the result. Memo indices
     * belong to one pickle; the stack is empty before and after. */
    val run()
    {
        stack.clear();
        marks.clear();
        memo.clear();
        for (;;) {
            const unsigned char op = *take(1);

            switch (op) {
            case 0x80: /* PROTO */
                take(1);
                break;
            case 0x95: /* FRAME */
                take(8);
                break;
            case '.': /* STOP */
            {
                val v = pop();
                if (!stack.empty() || !marks.empty())
                    fail("values left on the stack at STOP");
                return v;
            }
            case '(': /* MARK */
                marks.push_back(stack.size());
                break;
            case '0': /* POP */
                if (!marks.empty() && stack.size() == marks.back())
                    marks.pop_back();
                else
                    pop();
                break;
            case '1': /* POP_MARK */
                pop_mark();
                break;
            case '2': /* DUP */
                push(top());
                break;
            case 'N':
                push(mk(K_NONE));
                break;
            case 0x88: /* NEWTRUE */
            case 0x89: /* NEWFALSE */
            {
                val v = mk(K_BOOL);
                v->i = op == 0x88;
                push(v);
                break;
            }
            case 'I': /* INT (text; 01 / 00 are booleans) */
            {
                std::string s = line();
                if (s == "01" || s == "00") {
                    val v = mk(K_BOOL);
                    v->i = s == "01";
                    push(v);
                }
                else
                    push(integer(strtoll(s.c_str(), nullptr, 10)));
                break;
            }
            case 'L': /* LONG (text, trailing L) */
                push(integer(strtoll(line().c_str(), nullptr, 10)));
                break;
            case 'J': /* BININT */
                push(integer((int32_t)u(4)));
                break;
            case 'K': /* BININT1 */
                push(integer((long long)u(1)));
                break;
            case 'M': /* BININT2 */
                push(integer((long long)u(2)));
                break;
            case 0x8a: /* LONG1 */
                push(long_bytes(u(1)));
                break;
            case 0x8b: /* LONG4 */
                push(long_bytes(u(4)));
                break;
            case 'G': /* BINFLOAT, big-endian */
            {
                const unsigned char *b = take(8);
                uint64_t x = 0;
                val v = mk(K_FLOAT);

                for (int k = 0; k < 8; k++)
                    x = x << 8 | b[k];
                memcpy(&v->f, &x, 8);
                push(v);
                break;
            }
            case 'F': /* FLOAT (text) */
            {
                val v = mk(K_FLOAT);
                v->f = strtod(line().c_str(), nullptr);
                push(v);
                break;
            }
            case 'X': /* BINUNICODE */
            case 'T': /* BINSTRING */
            case 'B': /* BINBYTES */
            {
                const size_t n = u(4);
                push(str(take(n), n));
                break;
            }
            case 0x8c: /* SHORT_BINUNICODE */
            case 'U':  /* SHORT_BINSTRING */
            case 'C':  /* SHORT_BINBYTES */
            {
                const size_t n = u(1);
                push(str(take(n), n));
                break;
            }
            case 0x8d: /* BINUNICODE8 */
            case 0x8e: /* BINBYTES8 */
            case 0x96: /* BYTEARRAY8 */
            {
                const size_t n = u(8);
                push(str(take(n), n));
                break;
            }
            case 'S': /* STRING: quoted text */
            {
                std::string s = line();
                if (s.size() >= 2 && (s[0] == '\'' || s[0] == '"'))
                    s = s.substr(1, s.size() - 2);
                push(str((const unsigned char *)s.data(), s.size()));
                break;
            }
            case 'V': /* UNICODE: raw text line */
            {
                std::string s = line();
                push(str((const unsigned char *)s.data(), s.size()));
                break;
            }
            case ')':
                push(tuple({}));
                break;
            case 't':
                push(tuple(pop_mark()));
                break;
            case 0x85: /* TUPLE1 */
            case 0x86: /* TUPLE2 */
            case 0x87: /* TUPLE3 */
            {
                const int n = op - 0x84;
                std::vector<val> v(n);
                for (int k = n - 1; k >= 0; k--)
                    v[k] = pop();
                push(tuple(std::move(v)));
                break;
            }
            case ']':
                push(mk(K_LIST));
                break;
            case 'l': /* LIST */
            {
                val v = mk(K_LIST);
                v->items = pop_mark();
                push(v);
                break;
            }
            case 'a': /* APPEND */
            {
                val x = pop();
                val &l = top();
                if (l->k == K_LIST || l->k == K_SET)
                    l->items.push_back(x);
                break;
            }
            case 'e': /* APPENDS */
            case 0x90: /* ADDITEMS */
            {
                std::vector<val> xs = pop_mark();
                val &l = top();
                if (l->k == K_LIST || l->k == K_SET)
                    l->items.insert(l->items.end(), xs.begin(), xs.end());
                break;
            }
            case 0x8f: /* EMPTY_SET */
                push(mk(K_SET));
                break;
            case 0x91: /* FROZENSET */
            {
                val v = mk(K_SET);
                v->items = pop_mark();
                push(v);
                break;
            }
            case '}':
                push(mk(K_DICT));
                break;
            case 'd': /* DICT */
            {
                std::vector<val> kv = pop_mark();
                val d = mk(K_DICT);
                set_items(d, kv);
                push(d);
                break;
            }
            case 's': /* SETITEM */
            {
                val v = pop(), k = pop();
                set_items(top(), {k, v});
                break;
            }
            case 'u': /* SETITEMS */
            {
                std::vector<val> kv = pop_mark();
                set_items(top(), kv);
                break;
            }
            case 'c': /* GLOBAL "module\nname\n" */
            {
                val g = mk(K_GLOBAL);
                g->s = line();
                g->s2 = line();
                push(g);
                break;
            }
            case 0x93: /* STACK_GLOBAL */
            {
                val name = pop(), mod = pop();
                if (name->k != K_STR || mod->k != K_STR)
                    fail("STACK_GLOBAL without strings");
                val g = mk(K_GLOBAL);
                g->s = mod->s;
                g->s2 = name->s;
                push(g);
                break;
            }
            case 'R': /* REDUCE */
            {
                val args = pop(), fn = pop();
                push(reduce(fn, args));
                break;
            }
            case 0x81: /* NEWOBJ */
            {
                pop();
                pop();
                push(mk(K_OBJECT));
                break;
            }
            case 0x92: /* NEWOBJ_EX */
            {
                pop();
                pop();
                pop();
                push(mk(K_OBJECT));
                break;
            }
            case 'b': /* BUILD: the state does not change tensors or dicts */
                pop();
                top();
                break;
            case 'o': /* OBJ */
                pop_mark();
                push(mk(K_OBJECT));
                break;
            case 'i': /* INST */
                line();
                line();
                pop_mark();
                push(mk(K_OBJECT));
                break;
            case 'Q': /* BINPERSID */
                push(persistent(pop()));
                break;
            case 'P': /* PERSID (text id): not written by torch */
                fail("text persistent id");
            case 'p': /* PUT */
                memo[strtoll(line().c_str(), nullptr, 10)] = top();
                break;
            case 'q': /* BINPUT */
                memo[(long long)u(1)] = top();
                break;
            case 'r': /* LONG_BINPUT */
                memo[(long long)u(4)] = top();
                break;
            case 0x94: /* MEMOIZE */
                memo[(long long)memo.size()] = top();
                break;
            case 'g': /* GET */
            case 'h': /* BINGET */
            case 'j': /* LONG_BINGET */
            {
                const long long k = op == 'g'   ? strtoll(line().c_str(), nullptr, 10)
                                    : op == 'h' ? (long long)u(1)
                                                : (long long)u(4);
                auto it = memo.find(k);
                if (it == memo.end())
                    fail("memo key not found");
                push(it->second);
                break;
            }
            default:
                icoreg_fatal("Checkpoint <%s>: unsupported pickle opcode 0x%02x at "
                             "byte %ld",
                             path, op, (long)(p - 1 - base));
            }
        }
    }
};

bool holds_tensors(const val &d)
{
    if (d->k != K_DICT)
        return false;
    for (size_t k = 1; k < d->items.size(); k += 2)
        if (d->items[k]->k == K_TENSOR)
            return true;
    return false;
}

/* The state_dict inside the saved object, or null. */
val state_dict(const val &root)
{
    if (root->k != K_DICT)
        return nullptr;
    if (holds_tensors(root))
        return root;
    for (size_t k = 0; k + 1 < root->items.size(); k += 2) {
        const val &key = root->items[k], &v = root->items[k + 1];
        if (key->k == K_STR && (key->s == "model" || key->s == "state_dict") &&
            holds_tensors(v))
            return v;
    }
    val only;
    int n = 0;
    for (size_t k = 0; k + 1 < root->items.size(); k += 2)
        if (root->items[k]->k == K_STR && holds_tensors(root->items[k + 1])) {
            only = root->items[k + 1];
            n++;
        }
    return n == 1 ? only : nullptr;
}

struct storage_loc {
    long long off;
    long long bytes;
};

/* The index entries of the state_dict's float tensors, each checked to
 * lie inside its storage. */
void index_tensors(const file_ref &f, const val &sd,
                   const std::unordered_map<std::string, storage_loc> &where,
                   std::vector<struct pth_tensor> &ts)
{
    const char *path = f.path.c_str();

    for (size_t k = 1; k < sd->items.size(); k += 2) {
        const val &key = sd->items[k - 1], &tv = sd->items[k];

        if (tv->k != K_TENSOR || key->k != K_STR || tv->storage->dtype == PTH_OTHER)
            continue;
        auto it = where.find(tv->storage->s);
        if (it == where.end())
            icoreg_fatal("Checkpoint <%s>: storage <%s> of tensor <%s> is missing",
                         path, tv->storage->s.c_str(), key->s.c_str());
        struct pth_tensor t;
        long long last = tv->offset, numel = 1, ext, end;
        /* Shape, strides and offset come from the file: every extent is
         * computed with overflow checks, so that a crafted entry cannot
         * wrap past the storage bound below and index outside it later
         * (pth_read_f32's strided gather). */
        bool wrap = false;

        memset(&t, 0, sizeof(t));
        t.ndim = (int)tv->shape.size();
        t.storage_offset = (long)tv->offset;
        t.dtype = tv->storage->dtype;
        for (int d = 0; d < t.ndim; d++) {
            t.shape[d] = (long)tv->shape[d];
            t.stride[d] = (long)tv->stride[d];
            if (t.shape[d] <= 0 || t.stride[d] < 0)
                icoreg_fatal("Checkpoint <%s>: empty or negatively strided tensor "
                             "<%s>",
                             path, key->s.c_str());
            wrap |= __builtin_mul_overflow((long long)t.shape[d] - 1, (long long)t.stride[d],
                                           &ext);
            wrap |= __builtin_add_overflow(last, ext, &last);
            wrap |= __builtin_mul_overflow(numel, (long long)t.shape[d], &numel);
        }
        t.data_offset = (long)it->second.off;
        t.storage_bytes = (size_t)it->second.bytes;
        wrap |= __builtin_add_overflow(last, 1LL, &end);
        wrap |= __builtin_mul_overflow(end, (long long)elem_bytes(t.dtype), &end);
        wrap |= __builtin_mul_overflow(numel, (long long)sizeof(float), &ext);
        if (wrap || tv->offset < 0 || end > it->second.bytes)
            icoreg_fatal("Checkpoint <%s>: tensor <%s> exceeds its storage", path,
                         key->s.c_str());
        t.name = strdup(key->s.c_str());
        ts.push_back(t);
    }
}

void open_zip(const file_ref &f, std::vector<struct pth_tensor> &ts)
{
    const char *path = f.path.c_str();
    std::vector<zip_entry> es = zip_entries(f);
    const zip_entry *pkl = nullptr;

    /* The archive's root folder is named after the saved file. */
    for (const zip_entry &e : es) {
        const size_t n = e.name.size();
        if (n >= 8 && e.name.compare(n - 8, 8, "data.pkl") == 0 &&
            (n == 8 || e.name[n - 9] == '/')) {
            pkl = &e;
            break;
        }
    }
    if (!pkl)
        icoreg_fatal("Checkpoint <%s>: no data.pkl in the zip archive (not a "
                     "torch.save file)",
                     path);
    const std::string dir = pkl->name.substr(0, pkl->name.size() - 8) + "data/";
    std::unordered_map<std::string, storage_loc> where;

    for (const zip_entry &e : es)
        if (e.name.size() > dir.size() && e.name.compare(0, dir.size(), dir) == 0)
            where[e.name.substr(dir.size())] = {e.data, e.size};
    std::vector<unsigned char> buf = f.bytes(pkl->data, (size_t)pkl->size);
    unpickler m(buf, path);
    val sd = state_dict(m.run());

    if (!sd)
        icoreg_fatal("Checkpoint <%s>: no state_dict of tensors found", path);
    index_tensors(f, sd, where, ts);
}

void open_legacy(const file_ref &f, std::vector<struct pth_tensor> &ts)
{
    const char *path = f.path.c_str();
    std::vector<unsigned char> buf = f.bytes(0, (size_t)f.size);
    unpickler m(buf, path);
    std::unordered_map<std::string, storage_loc> where;

    /* The magic number 0x1950a86a20f9469cfc6c. */
    static const unsigned char magic[10] = {0x6c, 0xfc, 0x9c, 0x46, 0xf9,
                                            0x20, 0x6a, 0xa8, 0x50, 0x19};
    val mg = m.run();
    if (mg->k != K_BIGINT || mg->s.size() != 10 || memcmp(mg->s.data(), magic, 10) != 0)
        icoreg_fatal("Checkpoint <%s> is neither a zip archive nor a legacy "
                     "torch.save stream (no magic number)",
                     path);
    val ver = m.run();
    if (ver->k != K_INT || ver->i != 1001)
        icoreg_fatal("Checkpoint <%s> is neither a zip archive nor a legacy "
                     "torch.save stream (protocol %lld)",
                     path, ver->k == K_INT ? ver->i : -1LL);
    m.run(); /* system information */
    val sd = state_dict(m.run());
    val keys = m.run();
    if (keys->k != K_LIST)
        icoreg_fatal("Checkpoint <%s>: no storage key list after the object", path);
    long long off = m.p - buf.data();

    for (const val &key : keys->items) {
        int elsize = 0;

        if (key->k != K_STR)
            icoreg_fatal("Checkpoint <%s>: invalid storage key", path);
        for (const val &s : m.storages)
            if (s->s == key->s) {
                elsize = s->elsize;
                break;
            }
        if (!elsize)
            icoreg_fatal("Checkpoint <%s>: storage <%s> is used by no tensor", path,
                         key->s.c_str());
        if (off + 8 > f.size)
            icoreg_fatal("Checkpoint <%s>: truncated", path);
        const long long numel = (long long)le(&buf[off], 8);
        off += 8;
        if (numel < 0 || off + numel * elsize > f.size)
            icoreg_fatal("Checkpoint <%s>: truncated", path);
        where[key->s] = {off, numel * elsize};
        off += numel * elsize;
    }
    if (!sd)
        icoreg_fatal("Checkpoint <%s>: no state_dict of tensors found", path);
    index_tensors(f, sd, where, ts);
}

float half_to_float(uint16_t h)
{
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31,
                   m = h & 1023;
    uint32_t bits;
    float f;

    if (e == 0) {
        f = (float)m * (1.0f / 16777216.0f); /* m * 2^-24, exact */
        return s ? -f : f;
    }
    if (e == 31)
        bits = s | 0x7f800000u | (m << 13);
    else
        bits = s | ((e + 112) << 23) | (m << 13);
    memcpy(&f, &bits, 4);
    return f;
}

float to_float(const unsigned char *p, enum pth_dtype d)
{
    float f;
    uint32_t b;

    if (d == PTH_F32) {
        memcpy(&f, p, 4);
        return f;
    }
    if (d == PTH_F16)
        return half_to_float((uint16_t)le(p, 2));
    b = (uint32_t)le(p, 2) << 16;
    memcpy(&f, &b, 4);
    return f;
}

} // namespace

extern "C" void pth_open(struct pth_file *pf, const char *path)
{
    ICOREG_API_BEGIN
    file_ref f;
    unsigned char sig[4] = {0, 0, 0, 0};
    std::vector<struct pth_tensor> ts;

    memset(pf, 0, sizeof(*pf));
    f.path = path;
    if (!(f.fp = fopen(path, "rb")))
        icoreg_fatal("Unable to open checkpoint <%s>", path);
    fseeko(f.fp, 0, SEEK_END);
    f.size = (long long)ftello(f.fp);
    if (f.size < 8)
        icoreg_fatal("Checkpoint <%s> is too short", path);
    f.read_at(0, sig, 4);
    try {
        if (memcmp(sig, "PK\003\004", 4) == 0)
            open_zip(f, ts);
        else if (sig[0] == 0x80)
            open_legacy(f, ts);
        else
            open_safetensors(f, ts);
    }
    catch (...) {
        for (struct pth_tensor &t : ts)
            free(t.name);
        throw;
    }
    pf->fp = f.fp;
    f.fp = nullptr;
    pf->path = strdup(path);
    pf->ntensors = (int)ts.size();
    pf->tensors = (struct pth_tensor *)calloc(ts.size() + 1, sizeof(ts[0]));
    if (!ts.empty())
        memcpy(pf->tensors, ts.data(), ts.size() * sizeof(ts[0]));
    ICOREG_API_END
}

extern "C" const struct pth_tensor *pth_find(const struct pth_file *pf,
                                             const char *name)
{
    for (int i = 0; i < pf->ntensors; i++)
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
    t = pth_find(pf, name);
    if (!t)
        icoreg_fatal("Checkpoint <%s>: tensor <%s> not found", pf->path, name);
    if (t->ndim != ndim)
        icoreg_fatal("Checkpoint <%s>: tensor <%s> has %d dimensions, %d "
                     "expected",
                     pf->path, name, t->ndim, ndim);
    for (int d = 0; d < ndim; d++)
        if (shape[d] >= 0 && shape[d] != t->shape[d])
            icoreg_fatal("Checkpoint <%s>: tensor <%s> dimension %d is %ld, "
                         "%ld expected",
                         pf->path, name, d, t->shape[d], shape[d]);
    ICOREG_API_END_RET(t)
}

extern "C" int pth_strip_prefix(struct pth_file *pf, const char *prefix)
{
    const size_t n = strlen(prefix);
    int k = 0;

    for (int i = 0; i < pf->ntensors; i++)
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

    for (int d = 0; d < t->ndim; d++)
        n *= t->shape[d];
    return n;
}

extern "C" double pth_bytes(const struct pth_file *pf, const char *prefix)
{
    const size_t n = strlen(prefix);
    double s = 0;

    for (int i = 0; i < pf->ntensors; i++)
        if (strncmp(pf->tensors[i].name, prefix, n) == 0)
            s += (double)pth_numel(&pf->tensors[i]) * elem_bytes(pf->tensors[i].dtype);
    return s;
}

/* Contiguous tensors are read in one piece from their first element;
 * strided views read their storage's span and gather in C order. */
extern "C" float *pth_read_f32(const struct pth_file *pf,
                               const struct pth_tensor *t)
{
    float *out = NULL;
    ICOREG_API_BEGIN
    const long n = pth_numel(t);
    const size_t es = elem_bytes(t->dtype);
    long expect = 1, last = t->storage_offset;
    bool contiguous = true;

    if (t->dtype == PTH_OTHER)
        icoreg_fatal("Checkpoint <%s>: tensor <%s> is not a float tensor",
                     pf->path, t->name);
    for (int d = t->ndim - 1; d >= 0; d--) {
        if (t->shape[d] != 1 && t->stride[d] != expect)
            contiguous = false;
        expect *= t->shape[d];
        last += (t->shape[d] - 1) * t->stride[d];
    }
    const long first = t->storage_offset;
    const long span = contiguous ? n : last - first + 1;
    std::vector<unsigned char> raw((size_t)(span > 0 ? span : 1) * es);

    if ((size_t)(first + span) * es > t->storage_bytes ||
        fseeko(pf->fp, (off_t)(t->data_offset + (long long)first * (long long)es),
               SEEK_SET) != 0 ||
        fread(raw.data(), 1, (size_t)span * es, pf->fp) != (size_t)span * es)
        icoreg_fatal("Checkpoint <%s>: reading <%s> failed", pf->path, t->name);
    out = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    if (contiguous) {
        if (t->dtype == PTH_F32)
            memcpy(out, raw.data(), (size_t)n * 4);
        else
            for (long i = 0; i < n; i++)
                out[i] = to_float(&raw[(size_t)i * es], t->dtype);
    }
    else {
        long idx[PTH_MAX_DIMS] = {0};

        for (long i = 0; i < n; i++) {
            long off = 0;

            for (int d = 0; d < t->ndim; d++)
                off += idx[d] * t->stride[d];
            out[i] = to_float(&raw[(size_t)off * es], t->dtype);
            for (int d = t->ndim - 1; d >= 0; d--) {
                if (++idx[d] < t->shape[d])
                    break;
                idx[d] = 0;
            }
        }
    }
    ICOREG_API_END_RET(out)
}

extern "C" void pth_close(struct pth_file *pf)
{
    if (pf->fp)
        fclose(pf->fp);
    for (int i = 0; i < pf->ntensors; i++)
        free(pf->tensors[i].name);
    free(pf->tensors);
    free(pf->path);
    memset(pf, 0, sizeof(*pf));
}
