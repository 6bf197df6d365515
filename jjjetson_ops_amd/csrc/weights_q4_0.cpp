// On-disk Q4_0 weights: safetensors reader / writer that carries Q4_0 tensors
// beside F32 ones, the host fp32 -> Q4_0 quantizer, and the streaming converter
// (the offline repacker) from an F32 checkpoint to a Q4_0 one.
//
// The reference's loader reads F32 tensors only (WeightDtype, src/model/weight_loader.h:12-14;
// meta_to_host_tensor rejects every other dtype, src/model/safetensors_reader.cpp:349-355).
// The file layout is the standard one (8-byte little-endian header length, JSON
// header, data section; the same steps as safetensors_read_file,
// safetensors_reader.cpp:369-494).  A Q4_0 tensor of logical shape [rows, cols] is
// stored as dtype "U8", shape [rows, cols/32, 18] (the 18-byte block_q4_0 of the
// kernels, row-major), and is marked by the metadata entry
// "q4_0:<name>": "Q4_0", so stock safetensors readers load it as plain bytes.
// The GEMV/GEMM kernels read these blocks as they are: no further repacking.
#include <errno.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <map>
#include <string>
#include <thread>
#include <vector>

#include "jjjetson_ops_amd.h"

namespace jjo {
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
}  // namespace jjo

using jjo::clear_error;
using jjo::set_error;

namespace {

constexpr uint64_t kMaxHeaderBytes = 100u << 20;  // the format's own limit
const char *const kQ4Marker = "Q4_0";
const std::string kQ4KeyPrefix = "q4_0:";

// ------------------------------------------------------------------ Q4_0 rule
// Per 32 values: mx = the value of largest magnitude (the first on ties; only
// |v| > running max replaces it, so NaN never wins and all-zero blocks give +0),
// d = mx / -8 (stored fp16, nearest even), id = d != 0 ? 1/d : 0,
// nib = clamp((int)(v*id + 8.5), 0, 15) with the multiply and the add rounded
// separately.  ggml's quantize_row_q4_0 rule; the reference consumes such blocks
// (src/cuda/mm_q4_0_q8_1.cu:35-38,79-92).
#pragma clang fp contract(off)
void quantize_blocks(const float *w, uint8_t *out, int64_t n_blocks) {
    for (int64_t b = 0; b < n_blocks; ++b) {
        const float *v = w + b * JJO_QK4_0;
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < JJO_QK4_0; ++j) {
            const float a = std::fabs(v[j]);
            if (a > amax) {
                amax = a;
                mx = v[j];
            }
        }
        const float d = mx / -8.0f;
        const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
        uint8_t *o = out + b * JJO_BLOCK_Q4_0_BYTES;
        const _Float16 dh = (_Float16)d;
        memcpy(o, &dh, 2);
        for (int j = 0; j < 16; ++j) {
            int q[2];
            for (int h = 0; h < 2; ++h) {
                const float prod = v[j + 16 * h] * id;
                const float t = prod + 8.5f;
                // (int) truncates; NaN and values below 0 clamp to 0
                q[h] = (t >= 1.0f) ? std::min(15, (int)std::min(t, 16.0f)) : 0;
            }
            o[2 + j] = (uint8_t)(q[0] | (q[1] << 4));
        }
    }
}

int quantize_threads(const float *w, uint8_t *out, int64_t n_blocks, int num_threads) {
    if (num_threads <= 0) num_threads = (int)std::max(1u, std::thread::hardware_concurrency());
    const int64_t min_per_thread = 4096;  // blocks
    num_threads = (int)std::max<int64_t>(1, std::min<int64_t>(num_threads, n_blocks / min_per_thread));
    if (num_threads == 1) {
        quantize_blocks(w, out, n_blocks);
        return 0;
    }
    std::vector<std::thread> pool;
    const int64_t per = (n_blocks + num_threads - 1) / num_threads;
    for (int t = 0; t < num_threads; ++t) {
        const int64_t b0 = std::min(n_blocks, t * per), b1 = std::min(n_blocks, b0 + per);
        if (b1 <= b0) break;
        pool.emplace_back(quantize_blocks, w + b0 * JJO_QK4_0, out + b0 * JJO_BLOCK_Q4_0_BYTES, b1 - b0);
    }
    for (auto &th : pool) th.join();
    return 0;
}

// ------------------------------------------------------------------ JSON header
struct Meta {
    std::string name;
    std::string dtype;
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;
};

struct Header {
    std::vector<Meta> tensors;
    std::map<std::string, std::string> metadata;
};

class Json {
  public:
    Json(const char *p, size_t n) : p_(p), e_(p + n) {}
    bool ok() const { return err_.empty(); }
    const std::string &error() const { return err_; }

    bool parse_header(Header *h) {
        if (!expect('{')) return false;
        if (peek() == '}') return ++p_, true;
        for (;;) {
            std::string key;
            if (!string(&key) || !expect(':')) return false;
            if (key == "__metadata__") {
                if (!string_map(&h->metadata)) return false;
            } else {
                Meta m;
                m.name = key;
                if (!tensor(&m)) return false;
                h->tensors.push_back(std::move(m));
            }
            ws();
            if (p_ < e_ && *p_ == ',') { ++p_; continue; }
            return expect('}');
        }
    }
    bool at_end() {
        ws();
        return p_ == e_;
    }

  private:
    bool fail(const char *what) {
        if (err_.empty()) err_ = what;
        return false;
    }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    char peek() {
        ws();
        return p_ < e_ ? *p_ : '\0';
    }
    bool expect(char c) {
        ws();
        if (p_ >= e_ || *p_ != c) return fail("malformed JSON header");
        ++p_;
        return true;
    }
    static void put_utf8(std::string *s, uint32_t cp) {
        if (cp < 0x80) {
            s->push_back((char)cp);
        } else if (cp < 0x800) {
            s->push_back((char)(0xC0 | (cp >> 6)));
            s->push_back((char)(0x80 | (cp & 0x3F)));
        } else if (cp < 0x10000) {
            s->push_back((char)(0xE0 | (cp >> 12)));
            s->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            s->push_back((char)(0x80 | (cp & 0x3F)));
        } else {
            s->push_back((char)(0xF0 | (cp >> 18)));
            s->push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
            s->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            s->push_back((char)(0x80 | (cp & 0x3F)));
        }
    }
    bool hex4(uint32_t *v) {
        if (e_ - p_ < 4) return fail("truncated \\u escape");
        *v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            *v <<= 4;
            if (c >= '0' && c <= '9') *v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') *v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') *v |= (uint32_t)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool string(std::string *out) {
        if (!expect('"')) return false;
        out->clear();
        while (p_ < e_) {
            const char c = *p_++;
            if (c == '"') return true;
            if ((unsigned char)c < 0x20) return fail("control character in JSON string");
            if (c != '\\') {
                out->push_back(c);
                continue;
            }
            if (p_ >= e_) break;
            const char x = *p_++;
            switch (x) {
                case '"': out->push_back('"'); break;
                case '\\': out->push_back('\\'); break;
                case '/': out->push_back('/'); break;
                case 'b': out->push_back('\b'); break;
                case 'f': out->push_back('\f'); break;
                case 'n': out->push_back('\n'); break;
                case 'r': out->push_back('\r'); break;
                case 't': out->push_back('\t'); break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(&cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                        uint32_t lo;
                        if (e_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate");
                        p_ += 2;
                        if (!hex4(&lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: return fail("bad escape in JSON string");
            }
        }
        return fail("unterminated JSON string");
    }
    bool integer(int64_t *v) {
        ws();
        const char *s = p_;
        if (p_ < e_ && *p_ == '-') ++p_;
        const char *digits = p_;
        while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        if (p_ == digits || p_ - digits > 18) return fail("bad integer in JSON header");
        if (p_ < e_ && (*p_ == '.' || *p_ == 'e' || *p_ == 'E')) return fail("non-integer number in JSON header");
        *v = strtoll(std::string(s, p_).c_str(), nullptr, 10);
        return true;
    }
    bool int_array(std::vector<int64_t> *out) {
        if (!expect('[')) return false;
        out->clear();
        if (peek() == ']') return ++p_, true;
        for (;;) {
            int64_t v;
            if (!integer(&v)) return false;
            out->push_back(v);
            ws();
            if (p_ < e_ && *p_ == ',') { ++p_; continue; }
            return expect(']');
        }
    }
    bool string_map(std::map<std::string, std::string> *out) {
        if (!expect('{')) return false;
        if (peek() == '}') return ++p_, true;
        for (;;) {
            std::string k, v;
            if (!string(&k) || !expect(':') || !string(&v)) return false;
            (*out)[k] = v;
            ws();
            if (p_ < e_ && *p_ == ',') { ++p_; continue; }
            return expect('}');
        }
    }
    bool tensor(Meta *m) {
        if (!expect('{')) return false;
        bool has_dtype = false, has_shape = false, has_off = false;
        if (peek() != '}') {
            for (;;) {
                std::string key;
                if (!string(&key) || !expect(':')) return false;
                if (key == "dtype") {
                    if (!string(&m->dtype)) return false;
                    has_dtype = true;
                } else if (key == "shape") {
                    if (!int_array(&m->shape)) return false;
                    has_shape = true;
                } else if (key == "data_offsets") {
                    std::vector<int64_t> off;
                    if (!int_array(&off)) return false;
                    if (off.size() != 2 || off[0] < 0 || off[1] < off[0]) return fail("bad data_offsets");
                    m->begin = (uint64_t)off[0];
                    m->end = (uint64_t)off[1];
                    has_off = true;
                } else {
                    return fail("unknown key in tensor entry");
                }
                ws();
                if (p_ < e_ && *p_ == ',') { ++p_; continue; }
                break;
            }
        }
        if (!expect('}')) return false;
        if (!has_dtype || !has_shape || !has_off) return fail("tensor entry lacks dtype, shape or data_offsets");
        return true;
    }

    const char *p_;
    const char *e_;
    std::string err_;
};

void json_string(std::string *s, const std::string &v) {
    s->push_back('"');
    for (const char c : v) {
        switch (c) {
            case '"': *s += "\\\""; break;
            case '\\': *s += "\\\\"; break;
            case '\n': *s += "\\n"; break;
            case '\r': *s += "\\r"; break;
            case '\t': *s += "\\t"; break;
            default:
                if ((unsigned char)c < 0x20) {
                    char buf[8];
                    snprintf(buf, sizeof buf, "\\u%04x", (unsigned)(unsigned char)c);
                    *s += buf;
                } else {
                    s->push_back(c);
                }
        }
    }
    s->push_back('"');
}

// Header JSON for tensors laid out back to back in the given order; the result is
// padded with spaces to a multiple of 8 bytes (data section 8-byte aligned).
std::string make_header(const std::vector<Meta> &metas, const std::map<std::string, std::string> &metadata) {
    std::string s = "{";
    bool first = true;
    if (!metadata.empty()) {
        s += "\"__metadata__\":{";
        bool f2 = true;
        for (const auto &kv : metadata) {
            if (!f2) s += ",";
            f2 = false;
            json_string(&s, kv.first);
            s += ":";
            json_string(&s, kv.second);
        }
        s += "}";
        first = false;
    }
    for (const Meta &m : metas) {
        if (!first) s += ",";
        first = false;
        json_string(&s, m.name);
        s += ":{\"dtype\":";
        json_string(&s, m.dtype);
        s += ",\"shape\":[";
        for (size_t i = 0; i < m.shape.size(); ++i) {
            if (i) s += ",";
            s += std::to_string(m.shape[i]);
        }
        s += "],\"data_offsets\":[" + std::to_string(m.begin) + "," + std::to_string(m.end) + "]}";
    }
    s += "}";
    while ((8 + s.size()) % 8 != 0) s.push_back(' ');
    return s;
}

// ------------------------------------------------------------------ files
struct File {
    FILE *f = nullptr;
    ~File() {
        if (f) fclose(f);
    }
};

bool read_at(FILE *f, uint64_t off, void *dst, uint64_t n) {
    if (fseeko(f, (off_t)off, SEEK_SET) != 0) return false;
    return fread(dst, 1, n, f) == n;
}

bool shape_numel(const std::vector<int64_t> &shape, int64_t *numel) {
    int64_t n = 1;
    for (int64_t d : shape) {
        if (d < 0) return false;
        if (d != 0 && n > INT64_MAX / d) return false;
        n *= d;
    }
    *numel = n;
    return true;
}

// Opens `path` and parses its header.  data_base = file offset of the data section.
int open_and_parse(const char *path, File *file, Header *h, uint64_t *data_base, uint64_t *data_size) {
    file->f = fopen(path, "rb");
    if (file->f == nullptr) return set_error(JJO_ERR_INVALID_ARG, "cannot open %s: %s", path, strerror(errno));
    if (fseeko(file->f, 0, SEEK_END) != 0) return set_error(JJO_ERR_INVALID_ARG, "cannot seek %s", path);
    const off_t fsize = ftello(file->f);
    uint8_t len8[8];
    if (fsize < 8 || !read_at(file->f, 0, len8, 8))
        return set_error(JJO_ERR_INVALID_ARG, "%s: shorter than the 8-byte header length", path);
    uint64_t hs = 0;
    for (int i = 7; i >= 0; --i) hs = (hs << 8) | len8[i];
    if (hs > kMaxHeaderBytes || hs > (uint64_t)fsize - 8)
        return set_error(JJO_ERR_INVALID_ARG, "%s: header length %llu exceeds the file or the 100 MB limit", path,
                         (unsigned long long)hs);
    std::string text(hs, '\0');
    if (!read_at(file->f, 8, &text[0], hs)) return set_error(JJO_ERR_INVALID_ARG, "%s: cannot read header", path);
    Json js(text.data(), text.size());
    if (!js.parse_header(h) || !js.at_end())
        return set_error(JJO_ERR_INVALID_ARG, "%s: %s", path, js.ok() ? "trailing bytes after JSON header" : js.error().c_str());
    *data_base = 8 + hs;
    *data_size = (uint64_t)fsize - 8 - hs;
    for (const Meta &m : h->tensors)
        if (m.end > *data_size)
            return set_error(JJO_ERR_INVALID_ARG, "%s: tensor %s data_offsets [%llu, %llu) past the data section (%llu bytes)",
                             path, m.name.c_str(), (unsigned long long)m.begin, (unsigned long long)m.end,
                             (unsigned long long)*data_size);
    return JJO_OK;
}

// Logical description of one stored tensor (validates dtype and sizes).
int describe(const Header &h, const Meta &m, const char *path, int *dtype, std::vector<int64_t> *dims,
             int64_t *nbytes) {
    int64_t numel;
    if (!shape_numel(m.shape, &numel) || m.shape.empty() || m.shape.size() > 8)
        return set_error(JJO_ERR_INVALID_ARG, "%s: tensor %s has an unsupported shape", path, m.name.c_str());
    const auto it = h.metadata.find(kQ4KeyPrefix + m.name);
    const bool q4 = it != h.metadata.end() && it->second == kQ4Marker;
    if (m.dtype == "F32" && !q4) {
        if (numel > INT64_MAX / 4)
            return set_error(JJO_ERR_INVALID_ARG, "%s: tensor %s is too large", path, m.name.c_str());
        *dtype = JJO_WEIGHT_DTYPE_F32;
        *dims = m.shape;
        *nbytes = numel * 4;
    } else if (m.dtype == "U8" && q4) {
        if (m.shape.size() != 3 || m.shape[2] != JJO_BLOCK_Q4_0_BYTES)
            return set_error(JJO_ERR_INVALID_ARG, "%s: Q4_0 tensor %s must have shape [rows, cols/32, 18]", path,
                             m.name.c_str());
        if (m.shape[1] > INT64_MAX / JJO_QK4_0 || q4_0_bytes(m.shape[0], m.shape[1] * JJO_QK4_0) != numel)
            return set_error(JJO_ERR_INVALID_ARG, "%s: Q4_0 tensor %s has an unsupported shape", path,
                             m.name.c_str());
        *dtype = JJO_WEIGHT_DTYPE_Q4_0;
        *dims = {m.shape[0], m.shape[1] * JJO_QK4_0};
        *nbytes = numel;
    } else {
        return set_error(JJO_ERR_INVALID_ARG, "%s: unsupported dtype %s for tensor %s (F32, or U8 marked Q4_0)", path,
                         m.dtype.c_str(), m.name.c_str());
    }
    if ((uint64_t)*nbytes != m.end - m.begin)
        return set_error(JJO_ERR_INVALID_ARG, "%s: tensor %s holds %llu bytes, its shape needs %lld", path,
                         m.name.c_str(), (unsigned long long)(m.end - m.begin), (long long)*nbytes);
    return JJO_OK;
}

char *dup_string(const std::string &s) {
    char *p = (char *)malloc(s.size() + 1);
    if (p) memcpy(p, s.c_str(), s.size() + 1);
    return p;
}

int write_all(FILE *f, const void *p, size_t n, const char *path) {
    if (n && fwrite(p, 1, n, f) != n) return set_error(JJO_ERR_INVALID_ARG, "%s: write failed: %s", path, strerror(errno));
    return JJO_OK;
}

}  // namespace

extern "C" {

int64_t q4_0_bytes(int64_t rows, int64_t cols) {
    if (rows <= 0 || cols <= 0 || cols % JJO_QK4_0 != 0) return -1;
    if (rows > INT64_MAX / cols) return -1;
    return rows * (cols / JJO_QK4_0) * JJO_BLOCK_Q4_0_BYTES;
}

int quantize_q4_0_host(const float *w, void *out, int64_t rows, int64_t cols, int num_threads) {
    clear_error();
    if (w == nullptr || out == nullptr) return set_error(JJO_ERR_INVALID_ARG, "null pointer argument");
    if (q4_0_bytes(rows, cols) < 0)
        return set_error(JJO_ERR_INVALID_ARG, "rows (%lld) and cols (%lld) must be positive, cols a multiple of 32",
                         (long long)rows, (long long)cols);
    return quantize_threads(w, (uint8_t *)out, rows * (cols / JJO_QK4_0), num_threads);
}

void jjo_host_tensors_free(jjo_host_tensor *tensors, int num_tensors) {
    if (tensors == nullptr) return;
    for (int i = 0; i < num_tensors; ++i) {
        free(tensors[i].name);
        free(tensors[i].data);
        free(tensors[i].dims);
    }
    free(tensors);
}

const jjo_host_tensor *jjo_host_tensors_find(const jjo_host_tensor *tensors, int num_tensors, const char *name) {
    if (tensors == nullptr || name == nullptr) return nullptr;
    for (int i = 0; i < num_tensors; ++i)
        if (tensors[i].name != nullptr && strcmp(tensors[i].name, name) == 0) return &tensors[i];
    return nullptr;
}

int safetensors_read_file_q4_0(const char *path, jjo_host_tensor **out_tensors, int *out_num_tensors) {
    clear_error();
    if (path == nullptr || out_tensors == nullptr || out_num_tensors == nullptr)
        return set_error(JJO_ERR_INVALID_ARG, "null pointer argument");
    *out_tensors = nullptr;
    *out_num_tensors = 0;
    File file;
    Header h;
    uint64_t base, dsize;
    int rc = open_and_parse(path, &file, &h, &base, &dsize);
    if (rc != JJO_OK) return rc;
    const int n = (int)h.tensors.size();
    jjo_host_tensor *ts = (jjo_host_tensor *)calloc((size_t)std::max(n, 1), sizeof(jjo_host_tensor));
    if (ts == nullptr) return set_error(JJO_ERR_INVALID_ARG, "out of host memory");
    for (int i = 0; i < n; ++i) {
        const Meta &m = h.tensors[(size_t)i];
        int dtype;
        std::vector<int64_t> dims;
        int64_t nbytes;
        rc = describe(h, m, path, &dtype, &dims, &nbytes);
        if (rc == JJO_OK) {
            jjo_host_tensor &t = ts[i];
            t.name = dup_string(m.name);
            t.dims = (int64_t *)malloc(dims.size() * sizeof(int64_t));
            t.data = malloc((size_t)std::max<int64_t>(nbytes, 1));
            t.ndim = (int)dims.size();
            t.dtype = dtype;
            t.nbytes = nbytes;
            if (t.name == nullptr || t.dims == nullptr || t.data == nullptr) {
                rc = set_error(JJO_ERR_INVALID_ARG, "out of host memory reading %s", m.name.c_str());
            } else {
                memcpy(t.dims, dims.data(), dims.size() * sizeof(int64_t));
                if (!read_at(file.f, base + m.begin, t.data, (uint64_t)nbytes))
                    rc = set_error(JJO_ERR_INVALID_ARG, "%s: cannot read tensor %s", path, m.name.c_str());
            }
        }
        if (rc != JJO_OK) {
            jjo_host_tensors_free(ts, n);
            return rc;
        }
    }
    *out_tensors = ts;
    *out_num_tensors = n;
    return JJO_OK;
}

int safetensors_write_file_q4_0(const char *path, const jjo_host_tensor *tensors, int num_tensors) {
    clear_error();
    if (path == nullptr || (tensors == nullptr && num_tensors > 0) || num_tensors < 0)
        return set_error(JJO_ERR_INVALID_ARG, "null pointer or negative tensor count");
    std::vector<Meta> metas;
    std::map<std::string, std::string> metadata;
    uint64_t off = 0;
    for (int i = 0; i < num_tensors; ++i) {
        const jjo_host_tensor &t = tensors[i];
        if (t.name == nullptr || t.dims == nullptr || t.ndim <= 0 || t.ndim > 8 || (t.data == nullptr && t.nbytes > 0))
            return set_error(JJO_ERR_INVALID_ARG, "tensor %d: null name/dims/data or bad ndim", i);
        if (strncmp(t.name, "__metadata__", 13) == 0)
            return set_error(JJO_ERR_INVALID_ARG, "tensor name __metadata__ is reserved");
        for (int j = 0; j < i; ++j)
            if (strcmp(tensors[j].name, t.name) == 0) return set_error(JJO_ERR_INVALID_ARG, "duplicate tensor %s", t.name);
        Meta m;
        m.name = t.name;
        std::vector<int64_t> dims(t.dims, t.dims + t.ndim);
        int64_t numel;
        if (!shape_numel(dims, &numel)) return set_error(JJO_ERR_INVALID_ARG, "tensor %s: bad shape", t.name);
        int64_t need;
        if (t.dtype == JJO_WEIGHT_DTYPE_F32) {
            m.dtype = "F32";
            m.shape = dims;
            need = numel * 4;
        } else if (t.dtype == JJO_WEIGHT_DTYPE_Q4_0) {
            if (t.ndim != 2 || (need = q4_0_bytes(dims[0], dims[1])) < 0)
                return set_error(JJO_ERR_INVALID_ARG, "Q4_0 tensor %s must be [rows, cols] with cols %% 32 == 0", t.name);
            m.dtype = "U8";
            m.shape = {dims[0], dims[1] / JJO_QK4_0, JJO_BLOCK_Q4_0_BYTES};
            metadata[kQ4KeyPrefix + m.name] = kQ4Marker;
        } else {
            return set_error(JJO_ERR_INVALID_ARG, "tensor %s: unknown dtype %d", t.name, t.dtype);
        }
        if (t.nbytes != need)
            return set_error(JJO_ERR_INVALID_ARG, "tensor %s: nbytes %lld, shape needs %lld", t.name,
                             (long long)t.nbytes, (long long)need);
        m.begin = off;
        m.end = off + (uint64_t)need;
        off = m.end;
        metas.push_back(std::move(m));
    }
    const std::string hdr = make_header(metas, metadata);
    File file;
    file.f = fopen(path, "wb");
    if (file.f == nullptr) return set_error(JJO_ERR_INVALID_ARG, "cannot create %s: %s", path, strerror(errno));
    uint8_t len8[8];
    for (int i = 0; i < 8; ++i) len8[i] = (uint8_t)(((uint64_t)hdr.size() >> (8 * i)) & 0xff);
    int rc = write_all(file.f, len8, 8, path);
    if (rc == JJO_OK) rc = write_all(file.f, hdr.data(), hdr.size(), path);
    for (int i = 0; rc == JJO_OK && i < num_tensors; ++i) rc = write_all(file.f, tensors[i].data, (size_t)tensors[i].nbytes, path);
    if (rc == JJO_OK && fclose(file.f) != 0) rc = set_error(JJO_ERR_INVALID_ARG, "%s: close failed", path);
    file.f = nullptr;
    return rc;
}

int safetensors_quantize_q4_0(const char *in_path, const char *out_path, const char *const *names, int num_names,
                              int num_threads) {
    clear_error();
    if (in_path == nullptr || out_path == nullptr || (num_names > 0 && names == nullptr))
        return set_error(JJO_ERR_INVALID_ARG, "null pointer argument");
    File in;
    Header h;
    uint64_t base, dsize;
    int rc = open_and_parse(in_path, &in, &h, &base, &dsize);
    if (rc != JJO_OK) return rc;

    // Which tensors become Q4_0: the named ones (each must be a 2-D F32 tensor with
    // cols % 32 == 0), or with num_names < 0 every such tensor.
    std::vector<int> dtype(h.tensors.size());
    std::vector<std::vector<int64_t>> dims(h.tensors.size());
    std::vector<int64_t> nbytes(h.tensors.size());
    for (size_t i = 0; i < h.tensors.size(); ++i)
        if ((rc = describe(h, h.tensors[i], in_path, &dtype[i], &dims[i], &nbytes[i])) != JJO_OK) return rc;
    auto eligible = [&](size_t i) {
        return dtype[i] == JJO_WEIGHT_DTYPE_F32 && dims[i].size() == 2 && q4_0_bytes(dims[i][0], dims[i][1]) > 0;
    };
    std::vector<bool> conv(h.tensors.size(), false);
    if (num_names < 0) {
        for (size_t i = 0; i < h.tensors.size(); ++i) conv[i] = eligible(i);
    } else {
        for (int k = 0; k < num_names; ++k) {
            if (names[k] == nullptr) return set_error(JJO_ERR_INVALID_ARG, "names[%d] is NULL", k);
            size_t i = 0;
            while (i < h.tensors.size() && h.tensors[i].name != names[k]) ++i;
            if (i == h.tensors.size()) return set_error(JJO_ERR_INVALID_ARG, "%s: no tensor named %s", in_path, names[k]);
            if (!eligible(i))
                return set_error(JJO_ERR_INVALID_ARG, "tensor %s is not a 2-D F32 matrix with cols %% 32 == 0", names[k]);
            conv[i] = true;
        }
    }

    // Output header: file order kept, offsets recomputed; existing metadata kept
    // (Q4_0 tensors of the input stay Q4_0).
    std::vector<Meta> out_metas;
    std::map<std::string, std::string> out_md = h.metadata;
    uint64_t off = 0;
    for (size_t i = 0; i < h.tensors.size(); ++i) {
        Meta m = h.tensors[i];
        if (conv[i]) {
            m.dtype = "U8";
            m.shape = {dims[i][0], dims[i][1] / JJO_QK4_0, JJO_BLOCK_Q4_0_BYTES};
            out_md[kQ4KeyPrefix + m.name] = kQ4Marker;
        }
        const uint64_t n = conv[i] ? (uint64_t)q4_0_bytes(dims[i][0], dims[i][1]) : (uint64_t)nbytes[i];
        m.begin = off;
        m.end = off + n;
        off = m.end;
        out_metas.push_back(std::move(m));
    }
    const std::string hdr = make_header(out_metas, out_md);
    // Written to a temporary file beside out_path and renamed over it only once
    // complete: a failure leaves no partial output, and an existing out_path stays
    // intact until then.
    struct stat st_in, st_out;
    if (fstat(fileno(in.f), &st_in) == 0 && stat(out_path, &st_out) == 0 && st_in.st_dev == st_out.st_dev &&
        st_in.st_ino == st_out.st_ino)
        return set_error(JJO_ERR_INVALID_ARG, "%s: output path names the input file", out_path);
    const std::string tmp_path = std::string(out_path) + ".tmp" + std::to_string((long long)getpid());
    File out;
    out.f = fopen(tmp_path.c_str(), "wb");
    if (out.f == nullptr) return set_error(JJO_ERR_INVALID_ARG, "cannot create %s: %s", tmp_path.c_str(), strerror(errno));
    auto fail = [&](int code) {
        if (out.f != nullptr) fclose(out.f);
        out.f = nullptr;
        unlink(tmp_path.c_str());
        return code;
    };
    uint8_t len8[8];
    for (int i = 0; i < 8; ++i) len8[i] = (uint8_t)(((uint64_t)hdr.size() >> (8 * i)) & 0xff);
    if ((rc = write_all(out.f, len8, 8, out_path)) != JJO_OK) return fail(rc);
    if ((rc = write_all(out.f, hdr.data(), hdr.size(), out_path)) != JJO_OK) return fail(rc);
    // One tensor in memory at a time.
    std::vector<uint8_t> src, dst;
    for (size_t i = 0; i < h.tensors.size(); ++i) {
        const Meta &m = h.tensors[i];
        src.resize((size_t)nbytes[i]);
        if (!read_at(in.f, base + m.begin, src.data(), (uint64_t)nbytes[i]))
            return fail(set_error(JJO_ERR_INVALID_ARG, "%s: cannot read tensor %s", in_path, m.name.c_str()));
        if (conv[i]) {
            dst.resize((size_t)q4_0_bytes(dims[i][0], dims[i][1]));
            quantize_threads(reinterpret_cast<const float *>(src.data()), dst.data(),
                             dims[i][0] * (dims[i][1] / JJO_QK4_0), num_threads);
            rc = write_all(out.f, dst.data(), dst.size(), out_path);
        } else {
            rc = write_all(out.f, src.data(), src.size(), out_path);
        }
        if (rc != JJO_OK) return fail(rc);
    }
    const int close_rc = fclose(out.f);
    out.f = nullptr;
    if (close_rc != 0) return fail(set_error(JJO_ERR_INVALID_ARG, "%s: close failed", out_path));
    if (rename(tmp_path.c_str(), out_path) != 0)
        return fail(set_error(JJO_ERR_INVALID_ARG, "cannot rename %s to %s: %s", tmp_path.c_str(), out_path,
                              strerror(errno)));
    return JJO_OK;
}

}  // extern "C"
