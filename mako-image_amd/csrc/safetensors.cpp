// safetensors reader (the reference's safetensors::Files, as tests/safetensors_test.cpp:36-98 exercises it): one file
// or every *.safetensors file of a directory (a sharded checkpoint), and per tensor its dtype, its dims in GGUF order
// (dims[0] is the contiguous axis, the reverse of the header's "shape") and the absolute file offset of its data.
//
// File format (public safetensors specification): an 8-byte little-endian header length N, N bytes of JSON
//   {"name": {"dtype": "BF16", "shape": [rows, cols], "data_offsets": [begin, end]}, ..., "__metadata__": {...}}
// then the data, offsets relative to byte 8 + N. Everything in the header is checked against the file before a
// tensor is reported: offsets inside the data, end - begin = elements x element size, no duplicate names.
#include "common.hpp"

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <dirent.h>
#include <fcntl.h>
#include <memory>
#include <string>
#include <sys/stat.h>
#include <unistd.h>
#include <unordered_map>
#include <vector>

namespace mk {
namespace {

struct StTensor {
    std::string name, dtype_name;
    uint32_t dtype = MK_DTYPE_OTHER;
    std::vector<uint64_t> dims; // GGUF order
    uint32_t file = 0;
    uint64_t offset = 0, bytes = 0;
};

// Element size of each dtype the specification names (0: unknown).
uint64_t st_elem_size(const std::string& t, uint32_t* dtype)
{
    struct E {
        const char* name;
        uint64_t size;
        uint32_t dtype;
    };
    static const E table[] = {{"F64", 8, MK_DTYPE_OTHER},     {"F32", 4, MK_F32},         {"F16", 2, MK_F16},
                              {"BF16", 2, MK_BF16},           {"F8_E4M3", 1, MK_FP8_E4M3}, {"F8_E5M2", 1, MK_DTYPE_OTHER},
                              {"I64", 8, MK_DTYPE_OTHER},     {"U64", 8, MK_DTYPE_OTHER}, {"I32", 4, MK_DTYPE_OTHER},
                              {"U32", 4, MK_DTYPE_OTHER},     {"I16", 2, MK_DTYPE_OTHER}, {"U16", 2, MK_DTYPE_OTHER},
                              {"I8", 1, MK_DTYPE_OTHER},      {"U8", 1, MK_DTYPE_OTHER},  {"BOOL", 1, MK_DTYPE_OTHER}};
    for (const E& e : table)
        if (t == e.name) {
            *dtype = e.dtype;
            return e.size;
        }
    *dtype = MK_DTYPE_OTHER;
    return 0;
}

// A JSON reader for the header: objects, arrays, strings, numbers, true / false / null. Tensor entries keep dtype,
// shape and data_offsets; every other value is parsed and dropped.
struct Json {
    const char* p;
    const char* end;
    std::string err;

    bool fail(const char* what)
    {
        if (err.empty())
            err = what;
        return false;
    }
    void ws()
    {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r'))
            ++p;
    }
    bool lit(char c)
    {
        ws();
        if (p < end && *p == c) {
            ++p;
            return true;
        }
        return false;
    }
    bool str(std::string& out)
    {
        ws();
        if (p >= end || *p != '"')
            return fail("expected a string");
        ++p;
        out.clear();
        while (p < end && *p != '"') {
            char c = *p++;
            if (c == '\\') {
                if (p >= end)
                    return fail("bad escape");
                const char e = *p++;
                switch (e) {
                case '"': case '\\': case '/': out += e; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    if (end - p < 4)
                        return fail("bad \\u escape");
                    uint32_t cp = 0;
                    for (int i = 0; i < 4; ++i) {
                        const char h = *p++;
                        cp = cp * 16 + uint32_t(h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10
                                                : h >= 'A' && h <= 'F' ? h - 'A' + 10 : 99);
                        if (cp > 0xffff)
                            return fail("bad \\u escape");
                    }
                    // UTF-8 of a BMP code point (surrogate pairs are kept as two 3-byte sequences)
                    if (cp < 0x80)
                        out += char(cp);
                    else if (cp < 0x800) {
                        out += char(0xc0 | (cp >> 6));
                        out += char(0x80 | (cp & 63));
                    } else {
                        out += char(0xe0 | (cp >> 12));
                        out += char(0x80 | ((cp >> 6) & 63));
                        out += char(0x80 | (cp & 63));
                    }
                    break;
                }
                default: return fail("bad escape");
                }
            } else if (uint8_t(c) < 0x20) {
                return fail("control character in a string");
            } else {
                out += c;
            }
        }
        if (p >= end)
            return fail("unterminated string");
        ++p;
        return true;
    }
    // A non-negative integer (shapes and offsets); other numbers are parsed by skip().
    bool uint(uint64_t& v)
    {
        ws();
        if (p >= end || *p < '0' || *p > '9')
            return fail("expected a non-negative integer");
        v = 0;
        while (p < end && *p >= '0' && *p <= '9') {
            const uint64_t d = uint64_t(*p++ - '0');
            if (v > (UINT64_MAX - d) / 10)
                return fail("integer overflow");
            v = v * 10 + d;
        }
        if (p < end && (*p == '.' || *p == 'e' || *p == 'E'))
            return fail("expected an integer");
        return true;
    }
    bool uints(std::vector<uint64_t>& v)
    {
        v.clear();
        if (!lit('['))
            return fail("expected an array");
        if (lit(']'))
            return true;
        do {
            uint64_t x;
            if (!uint(x))
                return false;
            v.push_back(x);
        } while (lit(','));
        return lit(']') || fail("expected ']'");
    }
    bool skip(int depth = 0)
    {
        if (depth > 64)
            return fail("nesting too deep");
        ws();
        if (p >= end)
            return fail("unexpected end");
        if (*p == '"') {
            std::string s;
            return str(s);
        }
        if (*p == '{') {
            ++p;
            if (lit('}'))
                return true;
            do {
                std::string k;
                if (!str(k) || !lit(':') || !skip(depth + 1))
                    return fail("bad object");
            } while (lit(','));
            return lit('}') || fail("expected '}'");
        }
        if (*p == '[') {
            ++p;
            if (lit(']'))
                return true;
            do {
                if (!skip(depth + 1))
                    return false;
            } while (lit(','));
            return lit(']') || fail("expected ']'");
        }
        for (const char* w : {"true", "false", "null"}) {
            const size_t n = strlen(w);
            if (size_t(end - p) >= n && !memcmp(p, w, n)) {
                p += n;
                return true;
            }
        }
        const char* s = p;
        if (p < end && *p == '-')
            ++p;
        while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-'))
            ++p;
        return p > s || fail("unexpected character");
    }
};

} // namespace
} // namespace mk

using namespace mk;

struct mk_st {
    std::vector<std::string> paths;
    std::vector<int> fds;
    std::vector<StTensor> tensors;
    std::unordered_map<std::string, size_t> index;
    ~mk_st()
    {
        for (int fd : fds)
            if (fd >= 0)
                close(fd);
    }
};

namespace {

bool read_at(int fd, void* dst, uint64_t bytes, uint64_t off)
{
    char* d = static_cast<char*>(dst);
    while (bytes) {
        const ssize_t r = pread(fd, d, bytes > (1u << 30) ? (1u << 30) : size_t(bytes), off_t(off));
        if (r < 0 && errno == EINTR)
            continue;
        if (r <= 0)
            return false;
        d += r;
        off += uint64_t(r);
        bytes -= uint64_t(r);
    }
    return true;
}

mk_status parse_file(mk_st* st, uint32_t fi)
{
    const std::string& path = st->paths[fi];
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0)
        return fail(MK_ERR_ARG, "safetensors: cannot open " + path + ": " + strerror(errno));
    st->fds.push_back(fd);
    struct stat sb;
    if (fstat(fd, &sb) != 0)
        return fail(MK_ERR_ARG, "safetensors: cannot stat " + path);
    const uint64_t size = uint64_t(sb.st_size);
    uint8_t lenb[8];
    if (size < 8 || !read_at(fd, lenb, 8, 0))
        return fail(MK_ERR_ARG, "safetensors: " + path + ": shorter than its 8-byte header length");
    uint64_t n = 0;
    for (int i = 7; i >= 0; --i)
        n = (n << 8) | lenb[i];
    if (n < 2 || n > (uint64_t(100) << 20) || n > size - 8)
        return fail(MK_ERR_ARG, "safetensors: " + path + ": header length " + std::to_string(n) +
                                    " does not fit the file (" + std::to_string(size) + " bytes)");
    std::string hdr(size_t(n), '\0');
    if (!read_at(fd, hdr.data(), n, 8))
        return fail(MK_ERR_ARG, "safetensors: " + path + ": cannot read the header");
    const uint64_t data0 = 8 + n, data_size = size - data0;
    Json j{hdr.data(), hdr.data() + hdr.size(), {}};
    auto bad = [&](const std::string& what) {
        return fail(MK_ERR_ARG, "safetensors: " + path + ": " + what + (j.err.empty() ? "" : " (" + j.err + ")"));
    };
    if (!j.lit('{'))
        return bad("the header is not a JSON object");
    if (!j.lit('}')) {
        do {
            std::string name;
            if (!j.str(name) || !j.lit(':'))
                return bad("bad header entry");
            if (name == "__metadata__") {
                if (!j.skip())
                    return bad("bad __metadata__");
                continue;
            }
            StTensor t;
            t.name = name;
            t.file = fi;
            bool has_dtype = false, has_shape = false, has_off = false;
            std::vector<uint64_t> shape, offs;
            if (!j.lit('{'))
                return bad("tensor " + name + " is not an object");
            if (!j.lit('}')) {
                do {
                    std::string key;
                    if (!j.str(key) || !j.lit(':'))
                        return bad("tensor " + name + ": bad entry");
                    if (key == "dtype") {
                        if (!j.str(t.dtype_name))
                            return bad("tensor " + name + ": bad dtype");
                        has_dtype = true;
                    } else if (key == "shape") {
                        if (!j.uints(shape))
                            return bad("tensor " + name + ": bad shape");
                        has_shape = true;
                    } else if (key == "data_offsets") {
                        if (!j.uints(offs) || offs.size() != 2)
                            return bad("tensor " + name + ": data_offsets is not [begin, end]");
                        has_off = true;
                    } else if (!j.skip()) {
                        return bad("tensor " + name + ": bad value of " + key);
                    }
                } while (j.lit(','));
                if (!j.lit('}'))
                    return bad("tensor " + name + ": expected '}'");
            }
            if (!has_dtype || !has_shape || !has_off)
                return bad("tensor " + name + " lacks dtype, shape or data_offsets");
            if (shape.size() > MK_ST_MAX_DIMS)
                return bad("tensor " + name + " has more than " + std::to_string(MK_ST_MAX_DIMS) + " dims");
            const uint64_t es = st_elem_size(t.dtype_name, &t.dtype);
            if (!es)
                return bad("tensor " + name + ": unknown dtype " + t.dtype_name);
            uint64_t elems = 1;
            for (uint64_t d : shape) {
                if (d && elems > UINT64_MAX / d)
                    return bad("tensor " + name + ": shape overflows");
                elems *= d;
            }
            if (offs[0] > offs[1] || offs[1] > data_size)
                return bad("tensor " + name + ": data_offsets outside the file's data");
            if (elems > UINT64_MAX / es || offs[1] - offs[0] != elems * es)
                return bad("tensor " + name + ": " + std::to_string(offs[1] - offs[0]) + " bytes for " +
                           std::to_string(elems) + " elements of " + t.dtype_name);
            t.dims.assign(shape.rbegin(), shape.rend());
            t.offset = data0 + offs[0];
            t.bytes = offs[1] - offs[0];
            if (st->index.count(name))
                return bad("tensor " + name + " appears twice");
            st->index.emplace(name, st->tensors.size());
            st->tensors.push_back(std::move(t));
        } while (j.lit(','));
        if (!j.lit('}'))
            return bad("expected '}' at the end of the header");
    }
    j.ws();
    if (j.p != j.end)
        return bad("trailing bytes after the header object");
    return MK_OK;
}

void fill(const mk_st* st, const StTensor& t, mk_st_tensor* o)
{
    memset(o, 0, sizeof(*o));
    o->name = t.name.c_str();
    o->dtype_name = t.dtype_name.c_str();
    o->dtype = t.dtype;
    o->ndim = uint32_t(t.dims.size());
    for (size_t i = 0; i < t.dims.size(); ++i)
        o->dims[i] = t.dims[i];
    o->file = t.file;
    o->offset = t.offset;
    o->bytes = t.bytes;
    (void)st;
}

} // namespace

namespace mk {

const mk_st* st_lookup(const mk_st* st, const std::string& name, mk_st_tensor* t)
{
    auto it = st->index.find(name);
    if (it == st->index.end())
        return nullptr;
    fill(st, st->tensors[it->second], t);
    return st;
}

bool st_read(const mk_st* st, const mk_st_tensor& t, void* dst, uint64_t bytes, uint64_t off)
{
    return t.file < st->fds.size() && off + bytes <= t.bytes && read_at(st->fds[t.file], dst, bytes, t.offset + off);
}

} // namespace mk

extern "C" {

mk_status mk_st_open(const char* path, mk_st** out)
{
    if (!path || !out)
        return fail(MK_ERR_ARG, "st_open: null");
    *out = nullptr;
    auto st = std::make_unique<mk_st>();
    struct stat sb;
    if (stat(path, &sb) != 0)
        return fail(MK_ERR_ARG, std::string("safetensors: no such file or directory: ") + path);
    if (S_ISDIR(sb.st_mode)) {
        DIR* d = opendir(path);
        if (!d)
            return fail(MK_ERR_ARG, std::string("safetensors: cannot list ") + path);
        while (dirent* e = readdir(d)) {
            const std::string n = e->d_name;
            if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0)
                st->paths.push_back(std::string(path) + "/" + n);
        }
        closedir(d);
        std::sort(st->paths.begin(), st->paths.end());
        if (st->paths.empty())
            return fail(MK_ERR_ARG, std::string("safetensors: no *.safetensors file in ") + path);
    } else {
        st->paths.push_back(path);
    }
    for (uint32_t i = 0; i < st->paths.size(); ++i)
        MK_TRY(parse_file(st.get(), i));
    *out = st.release();
    return MK_OK;
}

mk_status mk_st_close(mk_st* st)
{
    delete st;
    return MK_OK;
}

mk_status mk_st_count(const mk_st* st, size_t* n, uint32_t* files)
{
    if (!st)
        return fail(MK_ERR_ARG, "st_count: null");
    if (n)
        *n = st->tensors.size();
    if (files)
        *files = uint32_t(st->paths.size());
    return MK_OK;
}

const char* mk_st_file_path(const mk_st* st, uint32_t file)
{
    return st && file < st->paths.size() ? st->paths[file].c_str() : nullptr;
}

mk_status mk_st_at(const mk_st* st, size_t i, mk_st_tensor* t)
{
    if (!st || !t)
        return fail(MK_ERR_ARG, "st_at: null");
    if (i >= st->tensors.size())
        return fail(MK_ERR_ARG, "st_at: index " + std::to_string(i) + " of " + std::to_string(st->tensors.size()));
    fill(st, st->tensors[i], t);
    return MK_OK;
}

mk_status mk_st_find(const mk_st* st, const char* name, mk_st_tensor* t)
{
    if (!st || !name || !t)
        return fail(MK_ERR_ARG, "st_find: null");
    if (!st_lookup(st, name, t))
        return fail(MK_ERR_ARG, std::string("safetensors: no tensor named ") + name);
    return MK_OK;
}

mk_status mk_st_read(const mk_st* st, const char* name, void* dst, size_t bytes)
{
    if (!st || !name || !dst)
        return fail(MK_ERR_ARG, "st_read: null");
    mk_st_tensor t;
    if (!st_lookup(st, name, &t))
        return fail(MK_ERR_ARG, std::string("safetensors: no tensor named ") + name);
    if (bytes != t.bytes)
        return fail(MK_ERR_ARG, std::string("st_read: ") + name + " holds " + std::to_string(t.bytes) + " bytes, not " +
                                    std::to_string(bytes));
    if (!st_read(st, t, dst, bytes, 0))
        return fail(MK_ERR_ARG, std::string("safetensors: cannot read ") + name);
    return MK_OK;
}

} // extern "C"
