// Packed B1_0 weights from .safetensors files: the host side of weight
// residency.  Replaces load_b1 (src/diffuser.cpp:39-50) over the mmap'd
// reader of src/safetensors.h:39-76.
//
// File format (safetensors): an 8-byte little-endian header length H, H
// bytes of JSON, then the tensor data.  The JSON object maps each tensor
// name to {"dtype": "...", "shape": [...], "data_offsets": [begin, end]}
// (offsets relative to the data section); an optional "__metadata__" entry
// holds string pairs.  A B1_0 tensor is U8 [out_dim, in_dim/32*6], as
// convert_to_b1_0_packed.py writes it.
#include <fcntl.h>
#include <stdint.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "bonsai_b1.h"

namespace {

// Read-only view of a whole file; unmapped on destruction.
struct Mapped {
    const uint8_t *p = nullptr;
    size_t n = 0;
    ~Mapped() {
        if (p) munmap(const_cast<uint8_t *>(p), n);
    }
    bool open(const char *path) {
        const int fd = ::open(path, O_RDONLY);
        if (fd < 0) return false;
        struct stat st;
        bool ok = fstat(fd, &st) == 0 && st.st_size > 0;
        if (ok) {
            void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
            ok = m != MAP_FAILED;
            if (ok) {
                p = static_cast<const uint8_t *>(m);
                n = (size_t)st.st_size;
            }
        }
        ::close(fd);
        return ok;
    }
};

// What the header says about one tensor.
struct Entry {
    std::string dtype;
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;
    bool has_offsets = false;
};

// Recursive-descent reader for the header JSON.  It descends only into the
// entry of the tensor asked for; every other value is parsed and skipped, so
// malformed JSON anywhere in the header is still an error.
class Header {
  public:
    Header(const char *s, size_t n) : s_(s), n_(n) {}

    // Finds `name` among the top-level keys.  Returns false on malformed JSON.
    bool find(const std::string &name, Entry *out, bool *found) {
        *found = false;
        ws();
        if (!eat('{')) return false;
        ws();
        if (peek() == '}') return ++i_, true;
        for (;;) {
            std::string key;
            ws();
            if (!str(&key)) return false;
            ws();
            if (!eat(':')) return false;
            ws();
            if (key == name) {
                if (!entry(out)) return false;
                *found = true;
            } else if (!skip()) {
                return false;
            }
            ws();
            if (eat(',')) continue;
            if (eat('}')) return true;
            return false;
        }
    }

  private:
    const char *s_;
    size_t n_, i_ = 0;
    int depth_ = 0;

    char peek() const { return i_ < n_ ? s_[i_] : '\0'; }
    bool eat(char c) {
        if (peek() != c) return false;
        ++i_;
        return true;
    }
    void ws() {
        while (i_ < n_ && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
    }
    bool str(std::string *out) {
        if (!eat('"')) return false;
        while (i_ < n_ && s_[i_] != '"') {
            char c = s_[i_++];
            if (c == '\\') {
                if (i_ >= n_) return false;
                const char e = s_[i_++];
                switch (e) {
                case '"': c = '"'; break;
                case '\\': c = '\\'; break;
                case '/': c = '/'; break;
                case 'b': c = '\b'; break;
                case 'f': c = '\f'; break;
                case 'n': c = '\n'; break;
                case 'r': c = '\r'; break;
                case 't': c = '\t'; break;
                case 'u': {
                    // \uXXXX, written back as UTF-8 (BMP code points only)
                    if (i_ + 4 > n_) return false;
                    unsigned v = 0;
                    for (int k = 0; k < 4; ++k) {
                        const char h = s_[i_++];
                        v <<= 4;
                        if (h >= '0' && h <= '9') v |= (unsigned)(h - '0');
                        else if (h >= 'a' && h <= 'f') v |= (unsigned)(h - 'a' + 10);
                        else if (h >= 'A' && h <= 'F') v |= (unsigned)(h - 'A' + 10);
                        else return false;
                    }
                    if (out) {
                        if (v < 0x80) {
                            out->push_back((char)v);
                        } else if (v < 0x800) {
                            out->push_back((char)(0xC0 | (v >> 6)));
                            out->push_back((char)(0x80 | (v & 0x3F)));
                        } else {
                            out->push_back((char)(0xE0 | (v >> 12)));
                            out->push_back((char)(0x80 | ((v >> 6) & 0x3F)));
                            out->push_back((char)(0x80 | (v & 0x3F)));
                        }
                    }
                    continue;
                }
                default: return false;
                }
            }
            if (out) out->push_back(c);
        }
        return eat('"');
    }
    // Non-negative integer (shapes and offsets).
    bool uint(uint64_t *v) {
        if (peek() < '0' || peek() > '9') return false;
        uint64_t x = 0;
        while (peek() >= '0' && peek() <= '9') {
            const uint64_t d = (uint64_t)(s_[i_++] - '0');
            if (x > (UINT64_MAX - d) / 10) return false;
            x = x * 10 + d;
        }
        *v = x;
        return true;
    }
    // Any JSON value, nested at most 64 deep.
    bool skip() {
        if (depth_ >= 64) return false;
        ++depth_;
        const bool ok = skip_value();
        --depth_;
        return ok;
    }
    bool skip_value() {
        const char c = peek();
        if (c == '{' || c == '[') {
            const char close = c == '{' ? '}' : ']';
            ++i_;
            ws();
            if (eat(close)) return true;
            for (;;) {
                ws();
                if (c == '{') {
                    if (!str(nullptr)) return false;
                    ws();
                    if (!eat(':')) return false;
                    ws();
                }
                if (!skip()) return false;
                ws();
                if (eat(',')) continue;
                return eat(close);
            }
        }
        if (c == '"') return str(nullptr);
        if (c == 't') return word("true");
        if (c == 'f') return word("false");
        if (c == 'n') return word("null");
        // number: sign, digits, fraction, exponent
        const size_t start = i_;
        if (peek() == '-') ++i_;
        while ((peek() >= '0' && peek() <= '9') || peek() == '.' || peek() == 'e' || peek() == 'E' ||
               peek() == '+' || peek() == '-')
            ++i_;
        return i_ > start;
    }
    bool word(const char *w) {
        const size_t k = strlen(w);
        if (n_ - i_ < k || strncmp(s_ + i_, w, k)) return false;
        i_ += k;
        return true;
    }
    bool uint_array(std::vector<uint64_t> *out) {
        if (!eat('[')) return false;
        ws();
        if (eat(']')) return true;
        for (;;) {
            ws();
            uint64_t v;
            if (!uint(&v)) return false;
            out->push_back(v);
            ws();
            if (eat(',')) continue;
            return eat(']');
        }
    }
    bool entry(Entry *e) {
        if (!eat('{')) return false;
        ws();
        if (eat('}')) return true;
        for (;;) {
            std::string key;
            ws();
            if (!str(&key)) return false;
            ws();
            if (!eat(':')) return false;
            ws();
            if (key == "dtype") {
                if (!str(&e->dtype)) return false;
            } else if (key == "shape") {
                std::vector<uint64_t> v;
                if (!uint_array(&v)) return false;
                for (uint64_t x : v) {
                    if (x > (uint64_t)INT64_MAX) return false;
                    e->shape.push_back((int64_t)x);
                }
            } else if (key == "data_offsets") {
                std::vector<uint64_t> v;
                if (!uint_array(&v) || v.size() != 2) return false;
                e->begin = v[0];
                e->end = v[1];
                e->has_offsets = true;
            } else if (!skip()) {
                return false;
            }
            ws();
            if (eat(',')) continue;
            return eat('}');
        }
    }
};

// Locates a B1_0 tensor: file bytes [*data, *data + *nbytes) with its dims.
int locate(const Mapped &m, const char *name, const uint8_t **data, uint64_t *nbytes, int64_t *rows,
           int64_t *cols) {
    if (m.n < 8) return BONSAI_B1_ERR_FORMAT;
    uint64_t hlen = 0;
    for (int k = 7; k >= 0; --k) hlen = (hlen << 8) | m.p[k];
    if (hlen == 0 || hlen > m.n - 8) return BONSAI_B1_ERR_FORMAT;
    Header h(reinterpret_cast<const char *>(m.p + 8), (size_t)hlen);
    Entry e;
    bool found = false;
    if (!h.find(name, &e, &found)) return BONSAI_B1_ERR_FORMAT;
    if (!found) return BONSAI_B1_ERR_NOT_FOUND;
    if (!e.has_offsets || e.shape.size() != 2 || e.end < e.begin) return BONSAI_B1_ERR_FORMAT;
    const uint64_t data_start = 8 + hlen;
    if (e.end > m.n - data_start) return BONSAI_B1_ERR_FORMAT;
    if (e.dtype != "U8" && e.dtype != "I8") return BONSAI_B1_ERR_FORMAT;
    const int64_t r = e.shape[0], c = e.shape[1];
    if (r <= 0 || c <= 0 || c % BONSAI_B1_BLOCK_BYTES) return BONSAI_B1_ERR_FORMAT;
    if ((uint64_t)r > (e.end - e.begin) / (uint64_t)c || (uint64_t)r * (uint64_t)c != e.end - e.begin)
        return BONSAI_B1_ERR_FORMAT;
    if (r > INT32_MAX || c / BONSAI_B1_BLOCK_BYTES * BONSAI_B1_BLOCK_SIZE > INT32_MAX) return BONSAI_B1_ERR_FORMAT;
    *data = m.p + data_start + e.begin;
    *nbytes = e.end - e.begin;
    *rows = r;
    *cols = c;
    return BONSAI_B1_OK;
}

} // namespace

extern "C" {

int bonsai_b1_safetensors_info(const char *path, const char *name, int *in_dim, int *out_dim,
                               uint64_t *data_offset, uint64_t *nbytes) {
    if (!path || !name) return BONSAI_B1_ERR_ARG;
    Mapped m;
    if (!m.open(path)) return BONSAI_B1_ERR_IO;
    const uint8_t *data = nullptr;
    uint64_t nb = 0;
    int64_t rows = 0, cols = 0;
    const int st = locate(m, name, &data, &nb, &rows, &cols);
    if (st != BONSAI_B1_OK) return st;
    if (in_dim) *in_dim = (int)(cols / BONSAI_B1_BLOCK_BYTES * BONSAI_B1_BLOCK_SIZE);
    if (out_dim) *out_dim = (int)rows;
    if (data_offset) *data_offset = (uint64_t)(data - m.p);
    if (nbytes) *nbytes = nb;
    return BONSAI_B1_OK;
}

int bonsai_b1_weights_load_safetensors(const char *path, const char *name, hipStream_t stream, B1Weights *out) {
    if (!path || !name || !out) return BONSAI_B1_ERR_ARG;
    Mapped m;
    if (!m.open(path)) return BONSAI_B1_ERR_IO;
    const uint8_t *data = nullptr;
    uint64_t nb = 0;
    int64_t rows = 0, cols = 0;
    int st = locate(m, name, &data, &nb, &rows, &cols);
    if (st != BONSAI_B1_OK) return st;
    st = bonsai_b1_weights_upload(data, (size_t)nb, (int)(cols / BONSAI_B1_BLOCK_BYTES * BONSAI_B1_BLOCK_SIZE),
                                  (int)rows, stream, out);
    if (st != BONSAI_B1_OK) return st;
    // The copy reads the mapping: finish it before the file is unmapped.
    if (hipStreamSynchronize(stream) != hipSuccess) {
        (void)bonsai_b1_weights_free(out);
        return BONSAI_B1_ERR_HIP;
    }
    return BONSAI_B1_OK;
}

} // extern "C"
