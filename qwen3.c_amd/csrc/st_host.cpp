// st_host.cpp - host side of the fmt=6 container reader: the safetensors header JSON, the
// shard index (c/st.h:200-339), the reads (c/st.h:171-195, 399-452) and the entry points of
// coli_hip_st_* that need no device.  The device loads are in container.hip.
#include "st_host.h"

#include <dirent.h>
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#include <algorithm>

namespace coli {

// ---------------------------------------------------------------- header JSON
// A strict reader for the safetensors header: objects, arrays, strings (escapes, \u as
// UTF-8), integers and the literals; nesting depth <= 16.  Numbers with a fraction or an
// exponent, or outside int64, are kept only as "not an integer" (metadata may hold them,
// shapes and offsets may not).
struct JVal {
    enum Kind { kNull, kBool, kInt, kNum, kStr, kArr, kObj } kind = kNull;
    int64_t i = 0;
    std::string s;
    std::vector<JVal> a;
    std::vector<std::pair<std::string, JVal>> o;
};

struct JParser {
    const char *p, *end;
    int depth = 0;
    bool ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
        return p < end;
    }
    static int hex(char c) {
        return c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10 : c >= 'A' && c <= 'F' ? c - 'A' + 10 : -1;
    }
    bool str(std::string &out) {
        if (p >= end || *p != '"') return false;
        p++;
        while (p < end && *p != '"') {
            unsigned char c = (unsigned char)*p++;
            if (c < 0x20) return false;
            if (c != '\\') {
                out.push_back((char)c);
                continue;
            }
            if (p >= end) return false;
            const char e = *p++;
            switch (e) {
            case '"': out.push_back('"'); break;
            case '\\': out.push_back('\\'); break;
            case '/': out.push_back('/'); break;
            case 'b': out.push_back('\b'); break;
            case 'f': out.push_back('\f'); break;
            case 'n': out.push_back('\n'); break;
            case 'r': out.push_back('\r'); break;
            case 't': out.push_back('\t'); break;
            case 'u': {
                if (end - p < 4) return false;
                unsigned cp = 0;
                for (int k = 0; k < 4; k++) {
                    const int h = hex(p[k]);
                    if (h < 0) return false;
                    cp = cp * 16 + (unsigned)h;
                }
                p += 4;
                if (cp >= 0xD800 && cp < 0xDC00) {   // surrogate pair
                    if (end - p < 6 || p[0] != '\\' || p[1] != 'u') return false;
                    unsigned lo = 0;
                    for (int k = 0; k < 4; k++) {
                        const int h = hex(p[2 + k]);
                        if (h < 0) return false;
                        lo = lo * 16 + (unsigned)h;
                    }
                    if (lo < 0xDC00 || lo >= 0xE000) return false;
                    p += 6;
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                } else if (cp >= 0xDC00 && cp < 0xE000) {
                    return false;
                }
                if (cp < 0x80) {
                    out.push_back((char)cp);
                } else if (cp < 0x800) {
                    out.push_back((char)(0xC0 | (cp >> 6)));
                    out.push_back((char)(0x80 | (cp & 63)));
                } else if (cp < 0x10000) {
                    out.push_back((char)(0xE0 | (cp >> 12)));
                    out.push_back((char)(0x80 | ((cp >> 6) & 63)));
                    out.push_back((char)(0x80 | (cp & 63)));
                } else {
                    out.push_back((char)(0xF0 | (cp >> 18)));
                    out.push_back((char)(0x80 | ((cp >> 12) & 63)));
                    out.push_back((char)(0x80 | ((cp >> 6) & 63)));
                    out.push_back((char)(0x80 | (cp & 63)));
                }
                break;
            }
            default: return false;
            }
        }
        if (p >= end) return false;
        p++;
        return true;
    }
    bool num(JVal &v) {
        bool neg = false, integral = true;
        if (p < end && *p == '-') {
            neg = true;
            p++;
        }
        if (p >= end || *p < '0' || *p > '9') return false;
        if (*p == '0' && p + 1 < end && p[1] >= '0' && p[1] <= '9') return false;   // no leading zeros
        uint64_t m = 0;
        bool ovf = false;
        while (p < end && *p >= '0' && *p <= '9') {
            const uint64_t d = (uint64_t)(*p++ - '0');
            if (m > (UINT64_MAX - d) / 10) ovf = true;
            else m = m * 10 + d;
        }
        if (p < end && *p == '.') {
            integral = false;
            p++;
            if (p >= end || *p < '0' || *p > '9') return false;
            while (p < end && *p >= '0' && *p <= '9') p++;
        }
        if (p < end && (*p == 'e' || *p == 'E')) {
            integral = false;
            p++;
            if (p < end && (*p == '+' || *p == '-')) p++;
            if (p >= end || *p < '0' || *p > '9') return false;
            while (p < end && *p >= '0' && *p <= '9') p++;
        }
        const uint64_t lim = neg ? (uint64_t)INT64_MAX + 1 : (uint64_t)INT64_MAX;
        if (integral && !ovf && m <= lim) {
            v.kind = JVal::kInt;
            v.i = neg ? (int64_t)(0 - m) : (int64_t)m;
        } else {
            v.kind = JVal::kNum;
        }
        return true;
    }
    bool lit(const char *w) {
        const size_t n = strlen(w);
        if ((size_t)(end - p) < n || memcmp(p, w, n)) return false;
        p += n;
        return true;
    }
    bool value(JVal &v) {
        if (!ws()) return false;
        if (*p == '{' || *p == '[') {
            if (++depth > 16) return false;
            const bool obj = *p == '{';
            p++;
            v.kind = obj ? JVal::kObj : JVal::kArr;
            if (!ws()) return false;
            if (*p == (obj ? '}' : ']')) {
                p++;
                depth--;
                return true;
            }
            for (;;) {
                if (obj) {
                    std::string k;
                    if (!ws() || !str(k) || !ws() || *p != ':') return false;
                    p++;
                    v.o.emplace_back(std::move(k), JVal());
                    if (!value(v.o.back().second)) return false;
                } else {
                    v.a.emplace_back();
                    if (!value(v.a.back())) return false;
                }
                if (!ws()) return false;
                if (*p == ',') {
                    p++;
                    continue;
                }
                if (*p == (obj ? '}' : ']')) {
                    p++;
                    depth--;
                    return true;
                }
                return false;
            }
        }
        if (*p == '"') {
            v.kind = JVal::kStr;
            return str(v.s);
        }
        if (*p == 't') {
            v.kind = JVal::kBool;
            v.i = 1;
            return lit("true");
        }
        if (*p == 'f') {
            v.kind = JVal::kBool;
            return lit("false");
        }
        if (*p == 'n') return lit("null");
        return num(v);
    }
};

static const JVal *jget(const JVal &o, const char *k) {
    for (const auto &kv : o.o)
        if (kv.first == k) return &kv.second;
    return nullptr;
}

// ---------------------------------------------------------------- shards
static bool st_err(const char *path, const char *what, const char *name = nullptr) {
    fprintf(stderr, "[HIP] container %s: %s%s%s\n", path, what, name ? " - tensor " : "", name ? name : "");
    return false;
}

// c/st.h:171-195: full pread in chunks of at most 1 GiB, EINTR retried, short reads named
bool pread_full(int fd, void *buf, int64_t n, int64_t off) {
    char *p = (char *)buf;
    int64_t got = 0;
    while (got < n) {
        const int64_t want = std::min<int64_t>(n - got, (int64_t)1 << 30);
        const ssize_t r = pread(fd, p + got, (size_t)want, (off_t)(off + got));
        if (r < 0) {
            if (errno == EINTR) continue;
            fprintf(stderr, "[HIP] container read: %s (offset %lld, %lld of %lld bytes)\n", strerror(errno),
                    (long long)off, (long long)got, (long long)n);
            return false;
        }
        if (r == 0) {
            fprintf(stderr, "[HIP] container read: end of file at offset %lld (%lld of %lld bytes)\n",
                    (long long)off, (long long)got, (long long)n);
            return false;
        }
        got += r;
    }
    return true;
}

static int dtype_code(const std::string &s) {
    if (s == "BF16") return kBF16;
    if (s == "F16") return kF16;
    if (s == "F32") return kF32;
    if (s == "U8" || s == "I8") return kU8;
    return -1;
}

// c/st.h:241-331: one shard's header into the index
bool index_shard(Shards &S, const std::string &path) {
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return st_err(path.c_str(), strerror(errno));
    S.fds.push_back(fd);
    S.paths.push_back(path);
    struct stat sb;
    if (fstat(fd, &sb) != 0) return st_err(path.c_str(), "fstat failed");
    const int64_t fsz = (int64_t)sb.st_size;
    uint64_t hlen = 0;
    if (fsz < 8 || !pread_full(fd, &hlen, 8, 0)) return st_err(path.c_str(), "no header length");
    if (hlen > (uint64_t)(fsz - 8) || hlen > kMaxHeader) return st_err(path.c_str(), "header length out of range");
    std::string hdr((size_t)hlen, '\0');
    if (!pread_full(fd, &hdr[0], (int64_t)hlen, 8)) return st_err(path.c_str(), "header read");
    JVal root;
    JParser jp{hdr.data(), hdr.data() + hdr.size()};
    if (!jp.value(root) || root.kind != JVal::kObj) return st_err(path.c_str(), "header is not a JSON object");
    jp.ws();
    if (jp.p != jp.end) return st_err(path.c_str(), "trailing bytes after the header object");
    const int64_t data0 = 8 + (int64_t)hlen;
    for (const auto &kv : root.o) {
        const std::string &name = kv.first;
        if (name == "__metadata__") continue;
        const JVal &m = kv.second;
        const JVal *dt = m.kind == JVal::kObj ? jget(m, "dtype") : nullptr;
        const JVal *of = m.kind == JVal::kObj ? jget(m, "data_offsets") : nullptr;
        const JVal *sh = m.kind == JVal::kObj ? jget(m, "shape") : nullptr;
        if (!dt || dt->kind != JVal::kStr || !of || of->kind != JVal::kArr || of->a.size() != 2 ||
            of->a[0].kind != JVal::kInt || of->a[1].kind != JVal::kInt || !sh || sh->kind != JVal::kArr)
            return st_err(path.c_str(), "malformed dtype / data_offsets / shape", name.c_str());
        const int64_t a0 = of->a[0].i, b0 = of->a[1].i;
        if (a0 < 0 || b0 < a0 || b0 > fsz - data0)
            return st_err(path.c_str(), "data_offsets outside the file", name.c_str());
        StTensor t;
        t.fd = fd;
        t.off = data0 + a0;
        t.nbytes = b0 - a0;
        t.dtype = dtype_code(dt->s);
        if (t.dtype < 0) return st_err(path.c_str(), "unsupported dtype", name.c_str());
        if (sh->a.size() > (size_t)kMaxDims) return st_err(path.c_str(), "too many dimensions", name.c_str());
        t.ndim = (int)sh->a.size();
        int64_t numel = 1;
        for (int k = 0; k < t.ndim; k++) {
            const JVal &d = sh->a[k];
            if (d.kind != JVal::kInt || d.i < 0 || (d.i != 0 && numel > INT64_MAX / d.i))
                return st_err(path.c_str(), "shape not a list of sizes, or its product overflows", name.c_str());
            t.shape[k] = d.i;
            numel *= d.i;
        }
        t.numel = numel;
        const int esz = t.dtype == kF32 ? 4 : t.dtype == kU8 ? 1 : 2;
        if (t.dtype != kU8 && t.nbytes != numel * esz)
            return st_err(path.c_str(), "element count disagrees with the byte span", name.c_str());
        S.map.emplace(name, t);   // an earlier shard's tensor of the same name stays
    }
    return true;
}

const StTensor *find(const Shards &S, const std::string &name) {
    const auto it = S.map.find(name);
    return it == S.map.end() ? nullptr : &it->second;
}

// ---------------------------------------------------------------- host conversions
static float bf16_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static float f16_f32(uint16_t h) {   // IEEE binary16 -> binary32, exact (subnormals, inf, NaN kept)
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    int e = (h >> 10) & 31;
    uint32_t m = h & 1023, u;
    if (e == 31) {
        u = sign | 0x7F800000u | (m << 13);
    } else if (e == 0) {
        if (!m) {
            u = sign;
        } else {   // subnormal: shift the mantissa up to an implicit 1
            int sh = 0;
            while (!(m & 1024)) {
                m <<= 1;
                sh++;
            }
            u = sign | (uint32_t)(127 - 15 + 1 - sh) << 23 | ((m & 1023) << 13);
        }
    } else {
        u = sign | (uint32_t)(e - 15 + 127) << 23 | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// the tensor's bytes as f32 into out[numel] (c/st.h:399-428)
bool read_f32(const StTensor &t, float *out) {
    if (t.dtype == kF32) return pread_full(t.fd, out, t.nbytes, t.off);
    if (t.dtype == kU8) return false;
    std::vector<uint16_t> raw((size_t)t.numel);
    if (!pread_full(t.fd, raw.data(), t.nbytes, t.off)) return false;
    for (int64_t i = 0; i < t.numel; i++) out[i] = t.dtype == kBF16 ? bf16_f32(raw[i]) : f16_f32(raw[i]);
    return true;
}

}  // namespace coli

using namespace coli;

// Index every *.safetensors file of dir (c/st.h:200-339).  NULL, with a message on stderr,
// when the directory has no shard or a shard's header breaks a rule above.
COLI_API ColiHipSt *coli_hip_st_open(const char *dir) {
    if (!dir) return nullptr;
    DIR *d = opendir(dir);
    if (!d) {
        fprintf(stderr, "[HIP] container %s: %s\n", dir, strerror(errno));
        return nullptr;
    }
    std::vector<std::string> files;
    while (const struct dirent *e = readdir(d)) {
        const size_t n = strlen(e->d_name);
        if (n > 12 && !strcmp(e->d_name + n - 12, ".safetensors")) files.push_back(std::string(dir) + "/" + e->d_name);
    }
    closedir(d);
    std::sort(files.begin(), files.end());
    if (files.empty()) {
        fprintf(stderr, "[HIP] container %s: no *.safetensors shard\n", dir);
        return nullptr;
    }
    ColiHipSt *st = new ColiHipSt();
    st->dir = dir;
    for (const auto &f : files)
        if (!index_shard(st->s, f)) {
            delete st;
            return nullptr;
        }
    return st;
}

COLI_API void coli_hip_st_close(ColiHipSt *st) { delete st; }

COLI_API int coli_hip_st_count(const ColiHipSt *st) { return st ? (int)st->s.map.size() : 0; }

// dtype (0 BF16, 1 F16, 2 F32, 3 U8/I8), element count, byte count and shape (up to 8
// dims) of a tensor; 0 when absent.
COLI_API int coli_hip_st_find(const ColiHipSt *st, const char *name, int *dtype, int64_t *numel, int64_t *nbytes,
                              int *ndim, int64_t *shape) {
    if (!st || !name) return 0;
    const StTensor *t = find(st->s, name);
    if (!t) return 0;
    if (dtype) *dtype = t->dtype;
    if (numel) *numel = t->numel;
    if (nbytes) *nbytes = t->nbytes;
    if (ndim) *ndim = t->ndim;
    if (shape)
        for (int k = 0; k < t->ndim; k++) shape[k] = t->shape[k];
    return 1;
}

// A float tensor (F32, BF16 or F16) as f32 into out, refusing more than cap elements
// (c/st.h:399-442); the element count, or -1.
COLI_API int64_t coli_hip_st_read_f32(const ColiHipSt *st, const char *name, float *out, int64_t cap) {
    if (!st || !name || !out) return -1;
    const StTensor *t = find(st->s, name);
    if (!t || t->dtype == kU8 || t->numel > cap) return -1;
    return read_f32(*t, out) ? t->numel : -1;
}

// Raw bytes of a tensor (U8 quantized data, c/st.h:445-452) into out, refusing more than
// cap bytes; the byte count, or -1.
COLI_API int64_t coli_hip_st_read_raw(const ColiHipSt *st, const char *name, void *out, int64_t cap) {
    if (!st || !name || !out) return -1;
    const StTensor *t = find(st->s, name);
    if (!t || t->nbytes > cap) return -1;
    return pread_full(t->fd, out, t->nbytes, t->off) ? t->nbytes : -1;
}
