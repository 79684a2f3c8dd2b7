// safetensors.cpp -- the .safetensors weight source of the linear layer, as
// the reference reads it (src/safetensor.pas:466-513 TSafeTensorFile.open,
// 584-683 getTensorDataMemBlock / getTensorDataMemBlockBF16), feeding the
// device weight upload instead of a host TMemoryBlock.
//
// Format: u64 little-endian header length H, H bytes of JSON, then the data
// block.  The JSON maps tensor names to {"dtype", "shape", "data_offsets":
// [begin, end)} with offsets relative to the data block; "__metadata__" (or
// any entry without data_offsets) is not a tensor.  Host code only.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cerrno>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/inv_hip.h"

extern "C" int inv_hip_internal_fail(int code, const char *msg);

namespace {

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return inv_hip_internal_fail(code, buf);
}

struct TensorInfo {
    std::string dtype;
    std::vector<int64_t> shape;
    int64_t begin = -1, end = -1;
};

// A JSON reader for safetensors headers: objects, arrays, strings (with the
// standard escapes), numbers, true/false/null.  Only tensor entries are kept.
class HeaderParser {
  public:
    HeaderParser(const char *s, size_t n) : p_(s), e_(s + n) {}

    bool parse(std::map<std::string, TensorInfo> &out, std::string &err) {
        ws();
        if (!eat('{')) return error(err, "header is not a JSON object");
        ws();
        if (eat('}')) return true;
        for (;;) {
            std::string key;
            ws();
            if (!str(key)) return error(err, "expected a tensor name");
            ws();
            if (!eat(':')) return error(err, "expected ':' after a name");
            ws();
            if (peek() == '{') {
                TensorInfo t;
                bool has_offsets = false;
                if (!tensor(t, has_offsets)) return error(err, "malformed entry for \"" + key + "\"");
                if (has_offsets) out[key] = t;
            } else if (!skip_value()) {
                return error(err, "malformed value for \"" + key + "\"");
            }
            ws();
            if (eat(',')) continue;
            if (eat('}')) break;
            return error(err, "expected ',' or '}'");
        }
        ws();
        return p_ == e_ ? true : error(err, "trailing bytes after the header object");
    }

  private:
    const char *p_, *e_;

    static bool error(std::string &err, const std::string &m) {
        err = m;
        return false;
    }
    char peek() const { return p_ < e_ ? *p_ : '\0'; }
    bool eat(char c) {
        if (p_ < e_ && *p_ == c) {
            ++p_;
            return true;
        }
        return false;
    }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }
    bool str(std::string &s) {
        if (!eat('"')) return false;
        while (p_ < e_ && *p_ != '"') {
            char c = *p_++;
            if (c == '\\') {
                if (p_ >= e_) return false;
                char x = *p_++;
                switch (x) {
                    case '"': s += '"'; break;
                    case '\\': s += '\\'; break;
                    case '/': s += '/'; break;
                    case 'b': s += '\b'; break;
                    case 'f': s += '\f'; break;
                    case 'n': s += '\n'; break;
                    case 'r': s += '\r'; break;
                    case 't': s += '\t'; break;
                    case 'u': {  // keep \uXXXX as UTF-8 (BMP only; names are ASCII in practice)
                        if (e_ - p_ < 4) return false;
                        unsigned v = 0;
                        for (int i = 0; i < 4; ++i) {
                            char h = *p_++;
                            v <<= 4;
                            if (h >= '0' && h <= '9') v |= (unsigned)(h - '0');
                            else if (h >= 'a' && h <= 'f') v |= (unsigned)(h - 'a' + 10);
                            else if (h >= 'A' && h <= 'F') v |= (unsigned)(h - 'A' + 10);
                            else return false;
                        }
                        if (v < 0x80) {
                            s += (char)v;
                        } else if (v < 0x800) {
                            s += (char)(0xC0 | (v >> 6));
                            s += (char)(0x80 | (v & 0x3F));
                        } else {
                            s += (char)(0xE0 | (v >> 12));
                            s += (char)(0x80 | ((v >> 6) & 0x3F));
                            s += (char)(0x80 | (v & 0x3F));
                        }
                        break;
                    }
                    default: return false;
                }
            } else {
                s += c;
            }
        }
        return eat('"');
    }
    bool integer(int64_t &v) {
        const char *b = p_;
        if (p_ < e_ && *p_ == '-') ++p_;
        while (p_ < e_ && isdigit((unsigned char)*p_)) ++p_;
        if (p_ == b || (p_ - b == 1 && *b == '-')) return false;
        if (p_ < e_ && (*p_ == '.' || *p_ == 'e' || *p_ == 'E')) return false;  // shapes and offsets are integers
        std::string t(b, p_);
        errno = 0;
        char *end = nullptr;
        long long x = strtoll(t.c_str(), &end, 10);
        if (errno || *end) return false;
        v = x;
        return true;
    }
    bool int_array(std::vector<int64_t> &a) {
        if (!eat('[')) return false;
        ws();
        if (eat(']')) return true;
        for (;;) {
            ws();
            int64_t v;
            if (!integer(v)) return false;
            a.push_back(v);
            ws();
            if (eat(',')) continue;
            return eat(']');
        }
    }
    bool tensor(TensorInfo &t, bool &has_offsets) {
        if (!eat('{')) return false;
        ws();
        if (eat('}')) return true;
        for (;;) {
            std::string k;
            ws();
            if (!str(k)) return false;
            ws();
            if (!eat(':')) return false;
            ws();
            if (k == "dtype") {
                if (!str(t.dtype)) return false;
            } else if (k == "shape") {
                if (!int_array(t.shape)) return false;
            } else if (k == "data_offsets") {
                std::vector<int64_t> o;
                if (!int_array(o) || o.size() != 2) return false;
                t.begin = o[0];
                t.end = o[1];
                has_offsets = true;
            } else if (!skip_value()) {
                return false;
            }
            ws();
            if (eat(',')) continue;
            return eat('}');
        }
    }
    // Nesting deeper than this is refused (a header that is only brackets
    // would otherwise recurse once per byte).
    static constexpr int kMaxDepth = 64;

    bool skip_value(int depth = 0) {
        if (depth > kMaxDepth) return false;
        ws();
        char c = peek();
        if (c == '"') {
            std::string s;
            return str(s);
        }
        if (c == '{' || c == '[') {
            const char open = c, close = (c == '{') ? '}' : ']';
            ++p_;
            ws();
            if (eat(close)) return true;
            for (;;) {
                ws();
                if (open == '{') {
                    std::string k;
                    if (!str(k)) return false;
                    ws();
                    if (!eat(':')) return false;
                }
                if (!skip_value(depth + 1)) return false;
                ws();
                if (eat(',')) continue;
                return eat(close);
            }
        }
        for (const char *lit : {"true", "false", "null"}) {
            const size_t n = strlen(lit);
            if ((size_t)(e_ - p_) >= n && !memcmp(p_, lit, n)) {
                p_ += n;
                return true;
            }
        }
        const char *b = p_;  // a number
        while (p_ < e_ && (isdigit((unsigned char)*p_) || strchr("+-.eE", *p_))) ++p_;
        return p_ != b;
    }
};

int dtype_size(const std::string &d) {
    if (d == "F32") return 4;
    if (d == "BF16" || d == "F16") return 2;
    return 0;
}

int dtype_code(const std::string &d) {
    if (d == "F32") return INV_DT_F32;
    if (d == "BF16") return INV_DT_BF16;
    if (d == "F16") return INV_DT_F16;
    return -1;
}

// A read-only private mapping of the whole file and its parsed header.
struct MappedFile {
    int fd = -1;
    void *base = MAP_FAILED;
    size_t size = 0;
    int64_t data_offset = 0;
    std::map<std::string, TensorInfo> tensors;

    ~MappedFile() {
        if (base != MAP_FAILED) munmap(base, size);
        if (fd >= 0) close(fd);
    }

    // Header checks follow TSafeTensorFile.open (src/safetensor.pas:479-507):
    // size > 7, header length < file size, every tensor inside the file.
    int open_file(const char *path, bool map_data) {
        if (!path) return fail(INV_ERR_ARG, "safetensors: null path");
        fd = ::open(path, O_RDONLY);
        if (fd < 0) return fail(INV_ERR_ARG, "safetensors: cannot open %s", path);
        struct stat st;
        if (fstat(fd, &st) != 0) return fail(INV_ERR_ARG, "safetensors: cannot stat %s", path);
        size = (size_t)st.st_size;
        if (size <= 8) return fail(INV_ERR_ARG, "safetensors: %s is too small (%zu bytes)", path, size);
        uint8_t hb[8];
        if (pread(fd, hb, 8, 0) != 8) return fail(INV_ERR_ARG, "safetensors: cannot read the header length");
        uint64_t h = 0;
        for (int i = 7; i >= 0; --i) h = (h << 8) | hb[i];
        if (h == 0 || h > size - 8) return fail(INV_ERR_ARG, "safetensors: invalid header length %llu", (unsigned long long)h);
        std::string json((size_t)h, '\0');
        if (pread(fd, &json[0], (size_t)h, 8) != (ssize_t)h) return fail(INV_ERR_ARG, "safetensors: truncated header");
        data_offset = 8 + (int64_t)h;
        std::string err;
        HeaderParser hp(json.data(), json.size());
        if (!hp.parse(tensors, err)) return fail(INV_ERR_ARG, "safetensors: bad header in %s: %s", path, err.c_str());
        const int64_t data_size = (int64_t)size - data_offset;
        for (auto &kv : tensors) {
            const TensorInfo &t = kv.second;
            if (t.begin < 0 || t.end < t.begin || t.end > data_size)
                return fail(INV_ERR_ARG, "safetensors: tensor \"%s\" lies outside the file (truncated?)", kv.first.c_str());
            const int es = dtype_size(t.dtype);
            if (es) {
                int64_t count = 1, bytes = 0;
                for (int64_t d : t.shape) {
                    if (d < 0) return fail(INV_ERR_ARG, "safetensors: tensor \"%s\" has a negative dimension", kv.first.c_str());
                    if (__builtin_mul_overflow(count, d, &count))
                        return fail(INV_ERR_ARG, "safetensors: tensor \"%s\": element count overflows", kv.first.c_str());
                }
                if (__builtin_mul_overflow(count, (int64_t)es, &bytes))
                    return fail(INV_ERR_ARG, "safetensors: tensor \"%s\": byte count overflows", kv.first.c_str());
                if (bytes != t.end - t.begin)
                    return fail(INV_ERR_ARG, "safetensors: tensor \"%s\" holds %lld bytes, its shape needs %lld",
                                kv.first.c_str(), (long long)(t.end - t.begin), (long long)bytes);
            }
        }
        if (map_data) {
            base = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
            if (base == MAP_FAILED) return fail(INV_ERR_OOM, "safetensors: cannot map %s", path);
        }
        return INV_OK;
    }

    const TensorInfo *find(const char *name) const {
        auto it = tensors.find(name ? name : "");
        return it == tensors.end() ? nullptr : &it->second;
    }
    const uint8_t *data(const TensorInfo &t) const { return (const uint8_t *)base + data_offset + t.begin; }
};

float half_to_float(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF, u;
    if (e == 0) {
        if (m == 0) {
            u = s;
        } else {  // subnormal half: normalise
            int sh = 0;
            while (!(m & 0x400)) {
                m <<= 1;
                ++sh;
            }
            m &= 0x3FF;
            u = s | ((uint32_t)(127 - 15 + 1 - sh) << 23) | (m << 13);
        }
    } else if (e == 31) {
        u = s | 0x7F800000u | (m << 13);
    } else {
        u = s | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// Tensor -> fp32 values (BF16 widened exactly, F16 widened exactly).
std::vector<float> to_f32(const uint8_t *src, const std::string &dtype, int64_t count) {
    std::vector<float> out((size_t)count);
    if (dtype == "F32") {
        memcpy(out.data(), src, (size_t)count * 4);
    } else if (dtype == "BF16") {
        for (int64_t i = 0; i < count; ++i) {
            uint16_t b;
            memcpy(&b, src + 2 * i, 2);
            uint32_t u = (uint32_t)b << 16;
            memcpy(&out[(size_t)i], &u, 4);
        }
    } else {
        for (int64_t i = 0; i < count; ++i) {
            uint16_t h;
            memcpy(&h, src + 2 * i, 2);
            out[(size_t)i] = half_to_float(h);
        }
    }
    return out;
}

}  // namespace

static int safetensors_info_impl(const char *path, const char *name, int *dtype, int *ndim, int64_t *shape,
                          int64_t *data_offset) {
    MappedFile f;
    int rc = f.open_file(path, false);
    if (rc != INV_OK) return rc;
    const TensorInfo *t = f.find(name);
    if (!t) return fail(INV_ERR_ARG, "safetensors: no tensor \"%s\" in %s", name ? name : "", path);
    if (dtype) *dtype = dtype_code(t->dtype);
    if (ndim) *ndim = (int)t->shape.size();
    if (shape)
        for (size_t i = 0; i < t->shape.size() && i < INV_ST_MAX_DIMS; ++i) shape[i] = t->shape[i];
    if (data_offset) *data_offset = f.data_offset + t->begin;
    return INV_OK;
}

static int weight_load_impl(const char *path, const char *name, const char *bias_name, int flags, inv_weight_t *out) {
    if (!out) return fail(INV_ERR_ARG, "safetensors: null output handle");
    *out = nullptr;
    MappedFile f;
    int rc = f.open_file(path, true);
    if (rc != INV_OK) return rc;
    const TensorInfo *t = f.find(name);
    if (!t) return fail(INV_ERR_ARG, "safetensors: no tensor \"%s\" in %s", name ? name : "", path);
    if (t->shape.size() != 2)
        return fail(INV_ERR_ARG, "safetensors: \"%s\" has %zu dimensions, a linear weight has 2 ([out x in])", name,
                    t->shape.size());
    if (!dtype_size(t->dtype))
        return fail(INV_ERR_UNSUPPORTED, "safetensors: \"%s\" has dtype %s (supported: BF16, F32, F16)", name,
                    t->dtype.c_str());
    const int64_t N = t->shape[0], K = t->shape[1];
    // the limits of the upload entry points, checked before any host conversion buffer is sized
    if (N <= 0 || K <= 0 || N > INT32_MAX / 2 || K > INT32_MAX / 2)
        return fail(INV_ERR_ARG, "safetensors: \"%s\" is %lld x %lld: each dimension must be in [1, 2^30)", name,
                    (long long)N, (long long)K);
    const bool gate_up = (flags & INV_ST_GATE_UP) != 0;
    if (gate_up && (N % 2))
        return fail(INV_ERR_ARG, "safetensors: \"%s\" has %lld rows, a fused gate|up weight needs an even count", name,
                    (long long)N);

    std::vector<float> bias;
    if (bias_name && *bias_name) {
        const TensorInfo *b = f.find(bias_name);
        if (!b) return fail(INV_ERR_ARG, "safetensors: no tensor \"%s\" in %s", bias_name, path);
        if (!dtype_size(b->dtype))
            return fail(INV_ERR_UNSUPPORTED, "safetensors: bias \"%s\" has dtype %s", bias_name, b->dtype.c_str());
        int64_t count = 1;
        for (int64_t d : b->shape) count *= d;
        if (count != N)
            return fail(INV_ERR_ARG, "safetensors: bias \"%s\" has %lld values, the weight has %lld rows", bias_name,
                        (long long)count, (long long)N);
        bias = to_f32(f.data(*b), b->dtype, count);
    }
    const float *bp = bias.empty() ? nullptr : bias.data();
    const uint8_t *src = f.data(*t);
    if (gate_up) {
        // [2F x K]: gate rows first, up rows second (src/quicknn_transformers.pas:595-597)
        const int64_t F = N / 2;
        std::vector<uint16_t> wb;
        const uint16_t *w16 = (const uint16_t *)src;
        if (t->dtype != "BF16") {
            std::vector<float> wf = to_f32(src, t->dtype, N * K);
            wb.resize((size_t)(N * K));
            for (int64_t i = 0; i < N * K; ++i) {
                uint32_t u;
                memcpy(&u, &wf[(size_t)i], 4);
                if (!(flags & INV_ST_TRUNCATE)) {
                    if ((u & 0x7fffffffu) > 0x7f800000u) u |= 0x00400000u;  // NaN stays NaN
                    else u += 0x7fffu + ((u >> 16) & 1u);
                }
                wb[(size_t)i] = (uint16_t)(u >> 16);
            }
            w16 = wb.data();
        }
        return inv_hip_weight_upload_gate_up(w16, w16 + F * K, F, K, bp, bp ? bp + F : nullptr, out);
    }
    if (t->dtype == "BF16") {
        // the mmap pointer straight into the upload, as getTensorDataMemBlockBF16
        // hands it to the reference (src/safetensor.pas:661-667)
        return inv_hip_weight_upload((const uint16_t *)src, N, K, bp, out);
    }
    if (t->dtype == "F32" && !(flags & INV_ST_TRUNCATE))
        return inv_hip_weight_upload_f32((const float *)src, N, K, bp, out);
    // F32 with INV_ST_TRUNCATE: the reference's SingleToBF16, u16 = u32 >> 16
    // (src/quicknn_common.pas:2010-2027, used at src/safetensor.pas:675);
    // F16: widened exactly, then rounded to bf16 (ties to even) or truncated.
    std::vector<float> w = (t->dtype == "F32") ? std::vector<float>() : to_f32(src, t->dtype, N * K);
    const float *wf = (t->dtype == "F32") ? (const float *)src : w.data();
    if (!(flags & INV_ST_TRUNCATE)) return inv_hip_weight_upload_f32(wf, N, K, bp, out);
    std::vector<uint16_t> wb((size_t)(N * K));
    for (int64_t i = 0; i < N * K; ++i) {
        uint32_t u;
        memcpy(&u, wf + i, 4);
        wb[(size_t)i] = (uint16_t)(u >> 16);
    }
    return inv_hip_weight_upload(wb.data(), N, K, bp, out);
}

// The C entry points: no exception crosses the ABI (an allocation failure in a
// host conversion buffer becomes INV_ERR_OOM, anything else INV_ERR_ARG).
extern "C" int inv_hip_safetensors_info(const char *path, const char *name, int *dtype, int *ndim, int64_t *shape,
                                        int64_t *data_offset) {
    try {
        return safetensors_info_impl(path, name, dtype, ndim, shape, data_offset);
    } catch (const std::bad_alloc &) {
        return fail(INV_ERR_OOM, "safetensors: host memory exhausted");
    } catch (const std::exception &e) {
        return fail(INV_ERR_ARG, "safetensors: %s", e.what());
    }
}

extern "C" int inv_hip_weight_load_safetensors(const char *path, const char *name, const char *bias_name, int flags,
                                               inv_weight_t *out) {
    try {
        return weight_load_impl(path, name, bias_name, flags, out);
    } catch (const std::bad_alloc &) {
        return fail(INV_ERR_OOM, "safetensors: host memory exhausted");
    } catch (const std::exception &e) {
        return fail(INV_ERR_ARG, "safetensors: %s", e.what());
    }
}
