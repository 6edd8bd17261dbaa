// safetensors reader: memory-maps a .safetensors file (or every shard named
// by a directory's model.safetensors.index.json) and indexes its header.
//
// Replaces src/safet.c (mda_safet_read / _tensor / _open_set / _find,
// :29-63, :147-163, :236-275).  Same file format and lookup semantics: an
// 8-byte little-endian header length, a JSON header mapping tensor names to
// {dtype, shape, data_offsets}, then the raw tensor bytes; a name missing from
// every shard is an error; offsets must lie inside the data section and match
// dtype x shape.  Differences: the header is parsed once into a table rather
// than searched with strstr per lookup, every safetensors dtype is indexed
// (the reference accepts BF16 and I64 only), and shards come from the index's
// weight_map instead of the "-of-N" file-name count.
//
// Host code only (no kernels); it links into librmda_moe.so beside the C ABI.
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"

namespace {

thread_local char g_st_msg[256] = "";

int st_fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_st_msg, sizeof(g_st_msg), fmt, ap);
    va_end(ap);
    return code;
}

struct StFile {
    void *map = nullptr;
    size_t mapped = 0;
    const uint8_t *data = nullptr;  // start of the data section
    uint64_t data_size = 0;
};

struct StEntry {
    std::string name;
    uint32_t file = 0;
    uint32_t dtype = RMDA_ST_OTHER;
    uint32_t ndim = 0;
    uint64_t shape[RMDA_ST_MAX_DIMS] = {0, 0, 0, 0};
    uint64_t begin = 0;
    uint64_t end = 0;
};

uint32_t dtype_code(const std::string &s) {
    if (s == "BF16") return RMDA_ST_BF16;
    if (s == "F16") return RMDA_ST_F16;
    if (s == "F32") return RMDA_ST_F32;
    if (s == "I64") return RMDA_ST_I64;
    if (s == "I32") return RMDA_ST_I32;
    if (s == "U8") return RMDA_ST_U8;
    return RMDA_ST_OTHER;
}

uint64_t dtype_bytes(uint32_t code) {
    switch (code) {
    case RMDA_ST_BF16:
    case RMDA_ST_F16: return 2;
    case RMDA_ST_F32:
    case RMDA_ST_I32: return 4;
    case RMDA_ST_I64: return 8;
    case RMDA_ST_U8: return 1;
    default: return 0;
    }
}

// ---- a small JSON reader for safetensors headers and index files ----
// Grammar: value = object | array | string | number | true | false | null.
// Strings keep ASCII; \uXXXX escapes below 0x80 decode, others become '?'
// (tensor names are ASCII in practice).  Depth is bounded.
struct Json {
    const char *p;
    const char *e;
    std::string err;

    void ws() {
        while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) {
            p += 1;
        }
    }
    bool fail(const char *what) {
        if (err.empty()) {
            err = what;
        }
        return false;
    }
    bool lit(char c) {
        ws();
        if (p < e && *p == c) {
            p += 1;
            return true;
        }
        return false;
    }
    bool str(std::string &out) {
        ws();
        if (p >= e || *p != '"') {
            return fail("expected a string");
        }
        p += 1;
        out.clear();
        while (p < e && *p != '"') {
            char c = *p++;
            if (c == '\\') {
                if (p >= e) {
                    return fail("bad escape");
                }
                char x = *p++;
                switch (x) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    if (e - p < 4) {
                        return fail("bad \\u escape");
                    }
                    unsigned v = 0;
                    for (int i = 0; i < 4; i += 1) {
                        char h = p[i];
                        v <<= 4;
                        if (h >= '0' && h <= '9') v |= (unsigned)(h - '0');
                        else if (h >= 'a' && h <= 'f') v |= (unsigned)(h - 'a' + 10);
                        else if (h >= 'A' && h <= 'F') v |= (unsigned)(h - 'A' + 10);
                        else return fail("bad \\u escape");
                    }
                    p += 4;
                    out += v < 0x80 ? (char)v : '?';
                    break;
                }
                default: return fail("bad escape");
                }
            } else {
                out += c;
            }
        }
        if (p >= e) {
            return fail("unterminated string");
        }
        p += 1;
        return true;
    }
    bool u64(uint64_t &v) {
        ws();
        if (p >= e || *p < '0' || *p > '9') {
            return fail("expected an unsigned integer");
        }
        v = 0;
        while (p < e && *p >= '0' && *p <= '9') {
            const uint64_t d = (uint64_t)(*p - '0');
            if (v > (UINT64_MAX - d) / 10) {
                return fail("integer overflow");
            }
            v = v * 10 + d;
            p += 1;
        }
        return true;
    }
    // skip any value
    bool skip(int depth = 0) {
        if (depth > 64) {
            return fail("nesting too deep");
        }
        ws();
        if (p >= e) {
            return fail("unexpected end");
        }
        if (*p == '"') {
            std::string s;
            return str(s);
        }
        if (*p == '{' || *p == '[') {
            const char close = *p == '{' ? '}' : ']';
            const bool obj = *p == '{';
            p += 1;
            if (lit(close)) {
                return true;
            }
            for (;;) {
                if (obj) {
                    std::string k;
                    if (!str(k) || !lit(':')) {
                        return fail("bad object");
                    }
                }
                if (!skip(depth + 1)) {
                    return false;
                }
                if (lit(close)) {
                    return true;
                }
                if (!lit(',')) {
                    return fail("expected ',' in container");
                }
            }
        }
        // number / literal
        const char *s = p;
        while (p < e && *p != ',' && *p != '}' && *p != ']' && *p != ' ' && *p != '\n' && *p != '\r' &&
               *p != '\t') {
            p += 1;
        }
        return p > s ? true : fail("bad value");
    }
};

// one header entry: {"dtype": "...", "shape": [...], "data_offsets": [a, b]}
bool parse_entry(Json &j, StEntry &t) {
    if (!j.lit('{')) {
        return j.fail("entry is not an object");
    }
    bool have_dtype = false;
    bool have_shape = false;
    bool have_offs = false;
    if (!j.lit('}')) {
        for (;;) {
            std::string k;
            if (!j.str(k) || !j.lit(':')) {
                return j.fail("bad entry key");
            }
            if (k == "dtype") {
                std::string v;
                if (!j.str(v)) {
                    return false;
                }
                t.dtype = dtype_code(v);
                have_dtype = true;
            } else if (k == "shape") {
                if (!j.lit('[')) {
                    return j.fail("shape is not an array");
                }
                t.ndim = 0;
                if (!j.lit(']')) {
                    for (;;) {
                        uint64_t v = 0;
                        if (!j.u64(v)) {
                            return false;
                        }
                        if (t.ndim == RMDA_ST_MAX_DIMS) {
                            return j.fail("more than 4 dimensions");
                        }
                        t.shape[t.ndim++] = v;
                        if (j.lit(']')) {
                            break;
                        }
                        if (!j.lit(',')) {
                            return j.fail("bad shape");
                        }
                    }
                }
                have_shape = true;
            } else if (k == "data_offsets") {
                if (!j.lit('[') || !j.u64(t.begin) || !j.lit(',') || !j.u64(t.end) || !j.lit(']')) {
                    return j.fail("bad data_offsets");
                }
                have_offs = true;
            } else if (!j.skip()) {
                return false;
            }
            if (j.lit('}')) {
                break;
            }
            if (!j.lit(',')) {
                return j.fail("expected ',' in entry");
            }
        }
    }
    return have_dtype && have_shape && have_offs ? true : j.fail("entry lacks dtype, shape or data_offsets");
}

}  // namespace

struct rmda_st {
    std::vector<StFile> files;
    std::vector<StEntry> entries;
    std::unordered_map<std::string, uint32_t> index;
};

namespace {

void st_unmap(rmda_st *st) {
    for (StFile &f : st->files) {
        if (f.map != nullptr) {
            munmap(f.map, f.mapped);
        }
    }
    st->files.clear();
}

int st_add_file(rmda_st *st, const std::string &path) {
    const int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) {
        return st_fail(RMDA_ERR_ARG, "%s: %s", path.c_str(), strerror(errno));
    }
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < 8) {
        close(fd);
        return st_fail(RMDA_ERR_ARG, "%s: not a safetensors file (too short)", path.c_str());
    }
    void *m = mmap(nullptr, (size_t)sb.st_size, PROT_READ, MAP_SHARED, fd, 0);
    close(fd);
    if (m == MAP_FAILED) {
        return st_fail(RMDA_ERR_ARG, "%s: cannot map", path.c_str());
    }
    StFile f;
    f.map = m;
    f.mapped = (size_t)sb.st_size;
    const uint8_t *bytes = static_cast<const uint8_t *>(m);
    uint64_t n = 0;
    memcpy(&n, bytes, 8);  // little endian on every supported host
    if (n > f.mapped - 8) {
        munmap(m, f.mapped);
        return st_fail(RMDA_ERR_ARG, "%s: not a safetensors file (header length %llu)", path.c_str(),
                       (unsigned long long)n);
    }
    f.data = bytes + 8 + n;
    f.data_size = f.mapped - 8 - n;
    const uint32_t fid = (uint32_t)st->files.size();
    st->files.push_back(f);

    Json j{reinterpret_cast<const char *>(bytes + 8), reinterpret_cast<const char *>(bytes + 8 + n), {}};
    if (!j.lit('{')) {
        return st_fail(RMDA_ERR_ARG, "%s: header is not a JSON object", path.c_str());
    }
    if (!j.lit('}')) {
        for (;;) {
            std::string name;
            if (!j.str(name) || !j.lit(':')) {
                return st_fail(RMDA_ERR_ARG, "%s: header: %s", path.c_str(), j.err.c_str());
            }
            if (name == "__metadata__") {
                if (!j.skip()) {
                    return st_fail(RMDA_ERR_ARG, "%s: header: %s", path.c_str(), j.err.c_str());
                }
            } else {
                StEntry t;
                t.name = name;
                t.file = fid;
                if (!parse_entry(j, t)) {
                    return st_fail(RMDA_ERR_ARG, "%s: %s: %s", path.c_str(), name.c_str(), j.err.c_str());
                }
                uint64_t elems = 1;
                for (uint32_t d = 0; d < t.ndim; d += 1) {
                    if (t.shape[d] != 0 && elems > UINT64_MAX / t.shape[d]) {
                        return st_fail(RMDA_ERR_ARG, "%s: %s: shape overflows", path.c_str(), name.c_str());
                    }
                    elems *= t.shape[d];
                }
                const uint64_t eb = dtype_bytes(t.dtype);
                if (t.end < t.begin || t.end > f.data_size || (eb != 0 && t.end - t.begin != elems * eb)) {
                    return st_fail(RMDA_ERR_ARG, "%s: %s: bad data offsets [%llu, %llu)", path.c_str(),
                                   name.c_str(), (unsigned long long)t.begin, (unsigned long long)t.end);
                }
                if (st->index.count(name) != 0) {
                    return st_fail(RMDA_ERR_ARG, "%s: %s: duplicate tensor name", path.c_str(), name.c_str());
                }
                st->index.emplace(name, (uint32_t)st->entries.size());
                st->entries.push_back(t);
            }
            if (j.lit('}')) {
                break;
            }
            if (!j.lit(',')) {
                return st_fail(RMDA_ERR_ARG, "%s: header: expected ','", path.c_str());
            }
        }
    }
    return RMDA_OK;
}

// model.safetensors.index.json: {"metadata": {...}, "weight_map": {name: file}}
int st_shards(const std::string &index_path, std::vector<std::string> &files) {
    FILE *fp = fopen(index_path.c_str(), "rb");
    if (fp == nullptr) {
        return st_fail(RMDA_ERR_ARG, "%s: %s", index_path.c_str(), strerror(errno));
    }
    std::string text;
    char buf[1 << 16];
    size_t got;
    while ((got = fread(buf, 1, sizeof(buf), fp)) > 0) {
        text.append(buf, got);
    }
    fclose(fp);
    Json j{text.data(), text.data() + text.size(), {}};
    if (!j.lit('{')) {
        return st_fail(RMDA_ERR_ARG, "%s: not a JSON object", index_path.c_str());
    }
    bool have_map = false;
    if (!j.lit('}')) {
        for (;;) {
            std::string k;
            if (!j.str(k) || !j.lit(':')) {
                return st_fail(RMDA_ERR_ARG, "%s: %s", index_path.c_str(), j.err.c_str());
            }
            if (k == "weight_map") {
                have_map = true;
                if (!j.lit('{')) {
                    return st_fail(RMDA_ERR_ARG, "%s: weight_map is not an object", index_path.c_str());
                }
                if (!j.lit('}')) {
                    for (;;) {
                        std::string name, file;
                        if (!j.str(name) || !j.lit(':') || !j.str(file)) {
                            return st_fail(RMDA_ERR_ARG, "%s: %s", index_path.c_str(), j.err.c_str());
                        }
                        bool seen = false;
                        for (const std::string &f : files) {
                            seen = seen || f == file;
                        }
                        if (!seen) {
                            files.push_back(file);
                        }
                        if (j.lit('}')) {
                            break;
                        }
                        if (!j.lit(',')) {
                            return st_fail(RMDA_ERR_ARG, "%s: weight_map: expected ','", index_path.c_str());
                        }
                    }
                }
            } else if (!j.skip()) {
                return st_fail(RMDA_ERR_ARG, "%s: %s", index_path.c_str(), j.err.c_str());
            }
            if (j.lit('}')) {
                break;
            }
            if (!j.lit(',')) {
                return st_fail(RMDA_ERR_ARG, "%s: expected ','", index_path.c_str());
            }
        }
    }
    if (!have_map || files.empty()) {
        return st_fail(RMDA_ERR_ARG, "%s: no weight_map entries", index_path.c_str());
    }
    return RMDA_OK;
}

}  // namespace

extern "C" {

int rmda_st_open(const char *path, rmda_st_t **out) {
    if (out == nullptr) {
        return st_fail(RMDA_ERR_ARG, "rmda_st_open: null out");
    }
    *out = nullptr;
    if (path == nullptr) {
        return st_fail(RMDA_ERR_ARG, "rmda_st_open: null path");
    }
    struct stat sb;
    if (stat(path, &sb) != 0) {
        return st_fail(RMDA_ERR_ARG, "%s: %s", path, strerror(errno));
    }
    rmda_st *st = new rmda_st();
    int rc = RMDA_OK;
    if (S_ISDIR(sb.st_mode)) {
        const std::string dir(path);
        const std::string index = dir + "/model.safetensors.index.json";
        struct stat ib;
        std::vector<std::string> files;
        if (stat(index.c_str(), &ib) == 0) {
            rc = st_shards(index, files);
        } else {
            files.push_back("model.safetensors");
        }
        for (size_t i = 0; rc == RMDA_OK && i < files.size(); i += 1) {
            rc = st_add_file(st, dir + "/" + files[i]);
        }
    } else {
        rc = st_add_file(st, std::string(path));
    }
    if (rc != RMDA_OK) {
        st_unmap(st);
        delete st;
        return rc;
    }
    *out = st;
    g_st_msg[0] = 0;
    return RMDA_OK;
}

void rmda_st_close(rmda_st_t *st) {
    if (st != nullptr) {
        st_unmap(st);
        delete st;
    }
}

const char *rmda_st_message(void) { return g_st_msg; }

uint32_t rmda_st_count(const rmda_st_t *st) { return st != nullptr ? (uint32_t)st->entries.size() : 0u; }

const char *rmda_st_name(const rmda_st_t *st, uint32_t i) {
    return st != nullptr && i < st->entries.size() ? st->entries[i].name.c_str() : nullptr;
}

int rmda_st_find(const rmda_st_t *st, const char *name, rmda_st_tensor_t *out) {
    if (st == nullptr || name == nullptr || out == nullptr) {
        return st_fail(RMDA_ERR_ARG, "rmda_st_find: null argument");
    }
    const auto it = st->index.find(name);
    if (it == st->index.end()) {
        return st_fail(RMDA_ERR_ARG, "safetensors: %s: missing", name);
    }
    const StEntry &t = st->entries[it->second];
    const StFile &f = st->files[t.file];
    memset(out, 0, sizeof(*out));
    out->data = f.data + t.begin;
    out->bytes = t.end - t.begin;
    out->dtype = t.dtype;
    out->ndim = t.ndim;
    for (uint32_t d = 0; d < t.ndim; d += 1) {
        out->shape[d] = t.shape[d];
    }
    out->file = t.file;
    return RMDA_OK;
}

}  // extern "C"
