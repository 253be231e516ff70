// safetensors reader: mmap + a small JSON parser for the header (objects,
// arrays, strings with escapes, integers, literals); everything the format
// allows in a header, nothing more.
#include "safetensors.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

#include "runtime.h"

namespace rfp4 {

namespace {

struct Json {
    const char *p, *end;
    bool ok = true;

    void ws()
    {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool eat(char c)
    {
        ws();
        if (p < end && *p == c) {
            p++;
            return true;
        }
        return false;
    }
    bool string(std::string *out)
    {
        ws();
        if (p >= end || *p != '"') return ok = false;
        p++;
        std::string s;
        while (p < end && *p != '"') {
            char c = *p++;
            if (c == '\\') {
                if (p >= end) return ok = false;
                char e = *p++;
                switch (e) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    if (end - p < 4) return ok = false;
                    unsigned v = 0;
                    for (int i = 0; i < 4; i++) {
                        char h = *p++;
                        v <<= 4;
                        if (h >= '0' && h <= '9') v |= (unsigned)(h - '0');
                        else if (h >= 'a' && h <= 'f') v |= (unsigned)(h - 'a' + 10);
                        else if (h >= 'A' && h <= 'F') v |= (unsigned)(h - 'A' + 10);
                        else return ok = false;
                    }
                    // names are ASCII in practice; keep other code points as UTF-8
                    if (v < 0x80) s += (char)v;
                    else if (v < 0x800) {
                        s += (char)(0xC0 | (v >> 6));
                        s += (char)(0x80 | (v & 0x3F));
                    } else {
                        s += (char)(0xE0 | (v >> 12));
                        s += (char)(0x80 | ((v >> 6) & 0x3F));
                        s += (char)(0x80 | (v & 0x3F));
                    }
                    break;
                }
                default: return ok = false;
                }
            } else {
                s += c;
            }
        }
        if (p >= end) return ok = false;
        p++; // closing quote
        if (out) *out = s;
        return true;
    }
    bool uint(uint64_t *out)
    {
        ws();
        if (p >= end || *p < '0' || *p > '9') return ok = false;
        uint64_t v = 0;
        while (p < end && *p >= '0' && *p <= '9') {
            uint64_t d = (uint64_t)(*p - '0');
            if (v > (UINT64_MAX - d) / 10) return ok = false;
            v = v * 10 + d;
            p++;
        }
        *out = v;
        return true;
    }
    bool uint_array(std::vector<uint64_t> *out)
    {
        if (!eat('[')) return ok = false;
        out->clear();
        if (eat(']')) return true;
        do {
            uint64_t v;
            if (!uint(&v)) return false;
            out->push_back(v);
        } while (eat(','));
        return eat(']') || (ok = false);
    }
    // any value, discarded
    bool skip(int depth = 0)
    {
        if (depth > 64) return ok = false;
        ws();
        if (p >= end) return ok = false;
        if (*p == '"') return string(nullptr);
        if (*p == '{') {
            p++;
            if (eat('}')) return true;
            do {
                if (!string(nullptr) || !eat(':') || !skip(depth + 1)) return ok = false;
            } while (eat(','));
            return eat('}') || (ok = false);
        }
        if (*p == '[') {
            p++;
            if (eat(']')) return true;
            do {
                if (!skip(depth + 1)) return false;
            } while (eat(','));
            return eat(']') || (ok = false);
        }
        const char *lits[] = {"true", "false", "null"};
        for (const char *l : lits) {
            size_t n = strlen(l);
            if ((size_t)(end - p) >= n && memcmp(p, l, n) == 0) {
                p += n;
                return true;
            }
        }
        if (*p == '-' || (*p >= '0' && *p <= '9')) {
            p++;
            while (p < end && (strchr("0123456789.eE+-", *p) != nullptr)) p++;
            return true;
        }
        return ok = false;
    }
};

} // namespace

StFile::~StFile()
{
    if (map_) munmap(map_, map_len_);
    if (fd_ >= 0) close(fd_);
}

uint32_t StFile::dtype_bytes(const std::string &d)
{
    if (d == "F64" || d == "I64" || d == "U64") return 8;
    if (d == "F32" || d == "I32" || d == "U32") return 4;
    if (d == "F16" || d == "BF16" || d == "I16" || d == "U16") return 2;
    if (d == "I8" || d == "U8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
    return 0;
}

int StFile::open(const char *path)
{
    if (!path) return set_error(RFP4_E_INVALID, "safetensors: null path");
    fd_ = ::open(path, O_RDONLY);
    if (fd_ < 0) return set_error(RFP4_E_INVALID, "safetensors: cannot open %s", path);
    struct stat sb;
    if (fstat(fd_, &sb) != 0 || sb.st_size < 8) return set_error(RFP4_E_SHAPE, "safetensors: %s is shorter than its header", path);
    map_len_ = (size_t)sb.st_size;
    void *m = mmap(nullptr, map_len_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (m == MAP_FAILED) {
        map_ = nullptr;
        return set_error(RFP4_E_INVALID, "safetensors: mmap of %s failed", path);
    }
    map_ = (uint8_t *)m;
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | map_[i];
    if (hlen > map_len_ - 8 || hlen > (100ull << 20))
        return set_error(RFP4_E_SHAPE, "safetensors: header length %llu does not fit the file", (unsigned long long)hlen);
    data_ = map_ + 8 + hlen;
    data_len_ = map_len_ - 8 - hlen;

    Json j{(const char *)map_ + 8, (const char *)map_ + 8 + hlen};
    if (!j.eat('{')) return set_error(RFP4_E_SHAPE, "safetensors: header is not a JSON object");
    if (!j.eat('}')) {
        do {
            std::string name;
            if (!j.string(&name) || !j.eat(':')) return set_error(RFP4_E_SHAPE, "safetensors: malformed header key");
            if (name == "__metadata__") {
                if (!j.skip()) return set_error(RFP4_E_SHAPE, "safetensors: malformed __metadata__");
                continue;
            }
            StTensor t;
            t.name = name;
            bool have_dtype = false, have_shape = false, have_off = false;
            if (!j.eat('{')) return set_error(RFP4_E_SHAPE, "safetensors: entry %s is not an object", name.c_str());
            if (!j.eat('}')) {
                do {
                    std::string key;
                    if (!j.string(&key) || !j.eat(':')) return set_error(RFP4_E_SHAPE, "safetensors: malformed entry %s", name.c_str());
                    if (key == "dtype") have_dtype = j.string(&t.dtype);
                    else if (key == "shape") have_shape = j.uint_array(&t.shape);
                    else if (key == "data_offsets") {
                        std::vector<uint64_t> off;
                        have_off = j.uint_array(&off) && off.size() == 2;
                        if (have_off) t.begin = off[0], t.end = off[1];
                    } else if (!j.skip()) {
                        return set_error(RFP4_E_SHAPE, "safetensors: malformed entry %s", name.c_str());
                    }
                    if (!j.ok) return set_error(RFP4_E_SHAPE, "safetensors: malformed entry %s", name.c_str());
                } while (j.eat(','));
                if (!j.eat('}')) return set_error(RFP4_E_SHAPE, "safetensors: unterminated entry %s", name.c_str());
            }
            if (!have_dtype || !have_shape || !have_off)
                return set_error(RFP4_E_SHAPE, "safetensors: entry %s lacks dtype, shape or data_offsets", name.c_str());
            const uint32_t eb = dtype_bytes(t.dtype);
            if (!eb) return set_error(RFP4_E_SHAPE, "safetensors: %s has unknown dtype %s", name.c_str(), t.dtype.c_str());
            if (t.begin > t.end || t.end > data_len_)
                return set_error(RFP4_E_SHAPE, "safetensors: %s lies outside the data section", name.c_str());
            if (t.end - t.begin != t.numel() * eb)
                return set_error(RFP4_E_SHAPE, "safetensors: %s holds %llu bytes, its shape needs %llu", name.c_str(),
                                 (unsigned long long)(t.end - t.begin), (unsigned long long)(t.numel() * eb));
            tensors_.push_back(t);
        } while (j.eat(','));
        if (!j.eat('}')) return set_error(RFP4_E_SHAPE, "safetensors: unterminated header");
    }
    return RFP4_OK;
}

const StTensor *StFile::find(const std::string &name) const
{
    for (const StTensor &t : tensors_)
        if (t.name == name) return &t;
    return nullptr;
}

float f16_to_f32_host(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else { // subnormal: normalise
            int e = -14;
            uint32_t m = mant;
            while (!(m & 0x400u)) {
                m <<= 1;
                e--;
            }
            bits = sign | ((uint32_t)(e + 127) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t f32_to_bf16_rne_host(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u)); // inf / nan
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

uint16_t f32_to_f16_rne_host(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint16_t)(sign | (a > 0x7F800000u ? 0x7E00u : 0x7C00u)); // nan, inf
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);                               // >= 65520: inf
    const int e = (int)(a >> 23) - 127;
    const uint32_t m = (a & 0x7FFFFFu) | 0x800000u; // 24-bit significand, value m * 2^(e-23)
    if (e < -14) {
        // subnormal: units of 2^-24, q = m * 2^(e+1), rounded to nearest even
        const int shift = -(e + 1);
        if (shift > 25) return (uint16_t)sign; // below 2^-25: rounds to zero
        const uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        return (uint16_t)(sign | (q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u)));
    }
    // normal: 10 fraction bits, the carry of the rounding may step the exponent
    const uint32_t q = ((uint32_t)(e + 15) << 10) | ((m >> 13) & 0x3FFu), rem = m & 0x1FFFu;
    return (uint16_t)(sign | (q + ((rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ? 1u : 0u)));
}

int StFile::read_f16(const StTensor &t, uint16_t *out, uint64_t count) const
{
    if (!out) return set_error(RFP4_E_INVALID, "safetensors: null output");
    const uint64_t n = t.numel();
    if (count < n) return set_error(RFP4_E_CAPACITY, "safetensors: %s needs %llu halves", t.name.c_str(), (unsigned long long)n);
    if (t.dtype == "F16") {
        memcpy(out, data(t), n * 2);
        return RFP4_OK;
    }
    std::vector<float> tmp(n);
    int rc = read_f32(t, tmp.data(), n);
    if (rc) return rc;
    for (uint64_t i = 0; i < n; i++) out[i] = f32_to_f16_rne_host(tmp[i]);
    return RFP4_OK;
}

int StFile::read_f32(const StTensor &t, float *out, uint64_t count) const
{
    if (!out) return set_error(RFP4_E_INVALID, "safetensors: null output");
    if (count < t.numel()) return set_error(RFP4_E_CAPACITY, "safetensors: %s needs %llu floats", t.name.c_str(), (unsigned long long)t.numel());
    const uint8_t *b = data(t);
    const uint64_t n = t.numel();
    if (t.dtype == "F32") {
        memcpy(out, b, n * 4);
    } else if (t.dtype == "BF16") {
        for (uint64_t i = 0; i < n; i++) {
            uint32_t bits = ((uint32_t)b[2 * i] | ((uint32_t)b[2 * i + 1] << 8)) << 16;
            memcpy(out + i, &bits, 4);
        }
    } else if (t.dtype == "F16") {
        for (uint64_t i = 0; i < n; i++) out[i] = f16_to_f32_host((uint16_t)(b[2 * i] | (b[2 * i + 1] << 8)));
    } else {
        return set_error(RFP4_E_SHAPE, "safetensors: %s has dtype %s (BF16, F16 or F32 expected)", t.name.c_str(), t.dtype.c_str());
    }
    return RFP4_OK;
}

} // namespace rfp4

// ---------------------------------------------------------------- C ABI
using namespace rfp4;

struct rfp4_st {
    StFile f;
};

extern "C" {

int rfp4_st_open(const char *path, rfp4_st **out)
{
    if (!out) return set_error(RFP4_E_INVALID, "rfp4_st_open: null output");
    *out = nullptr;
    rfp4_st *st = new rfp4_st();
    int rc = st->f.open(path);
    if (rc) {
        delete st;
        return rc;
    }
    *out = st;
    return RFP4_OK;
}

int rfp4_st_close(rfp4_st *st)
{
    delete st;
    return RFP4_OK;
}

int rfp4_st_count(const rfp4_st *st, uint32_t *count)
{
    if (!st || !count) return set_error(RFP4_E_INVALID, "rfp4_st_count: null argument");
    *count = (uint32_t)st->f.tensors().size();
    return RFP4_OK;
}

int rfp4_st_name(const rfp4_st *st, uint32_t i, const char **name)
{
    if (!st || !name) return set_error(RFP4_E_INVALID, "rfp4_st_name: null argument");
    if (i >= st->f.tensors().size()) return set_error(RFP4_E_INVALID, "rfp4_st_name: index %u out of range", i);
    *name = st->f.tensors()[i].name.c_str();
    return RFP4_OK;
}

int rfp4_st_info(const rfp4_st *st, const char *name, char dtype[8], uint32_t *ndim, uint64_t shape[8], uint64_t *nbytes)
{
    if (!st || !name) return set_error(RFP4_E_INVALID, "rfp4_st_info: null argument");
    const StTensor *t = st->f.find(name);
    if (!t) return set_error(RFP4_E_INVALID, "rfp4_st_info: no tensor %s", name);
    if (t->shape.size() > 8) return set_error(RFP4_E_SHAPE, "rfp4_st_info: %s has %zu dimensions", name, t->shape.size());
    if (dtype) {
        memset(dtype, 0, 8);
        strncpy(dtype, t->dtype.c_str(), 7);
    }
    if (ndim) *ndim = (uint32_t)t->shape.size();
    if (shape)
        for (size_t i = 0; i < t->shape.size(); i++) shape[i] = t->shape[i];
    if (nbytes) *nbytes = t->end - t->begin;
    return RFP4_OK;
}

int rfp4_st_read_f32(const rfp4_st *st, const char *name, float *out, uint64_t count)
{
    if (!st || !name) return set_error(RFP4_E_INVALID, "rfp4_st_read_f32: null argument");
    const StTensor *t = st->f.find(name);
    if (!t) return set_error(RFP4_E_INVALID, "rfp4_st_read_f32: no tensor %s", name);
    return st->f.read_f32(*t, out, count);
}

int rfp4_st_read_f16(const rfp4_st *st, const char *name, uint16_t *out, uint64_t count)
{
    if (!st || !name) return set_error(RFP4_E_INVALID, "rfp4_st_read_f16: null argument");
    const StTensor *t = st->f.find(name);
    if (!t) return set_error(RFP4_E_INVALID, "rfp4_st_read_f16: no tensor %s", name);
    return st->f.read_f16(*t, out, count);
}

} // extern "C"
