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

#include <algorithm>
#include <string>
#include <thread>
#include <unordered_map>
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

    // Every top-level entry but "__metadata__", in header order.  Returns
    // false on malformed JSON or a repeated name.
    bool index(std::vector<std::pair<std::string, Entry>> *out) {
        ws();
        if (!eat('{')) return false;
        ws();
        if (peek() == '}') return ++i_, true;
        std::unordered_map<std::string, int> seen;
        for (;;) {
            std::string key;
            ws();
            if (!str(&key)) return false;
            ws();
            if (!eat(':')) return false;
            ws();
            if (key == "__metadata__") {
                if (!skip()) return false;
            } else {
                Entry e;
                if (!entry(&e) || !seen.emplace(key, 0).second) return false;
                out->emplace_back(std::move(key), std::move(e));
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

// A B1_0 tensor is U8 (or I8) [rows, cols], cols a whole number of 6-byte
// blocks, its byte range inside the data section (data_len bytes) and
// consistent with the shape.
int b1_check(const Entry &e, uint64_t data_len, int64_t *rows, int64_t *cols) {
    if (!e.has_offsets || e.shape.size() != 2 || e.end < e.begin) return BONSAI_B1_ERR_FORMAT;
    if (e.end > data_len) return BONSAI_B1_ERR_FORMAT;
    if (e.dtype != "U8" && e.dtype != "I8") return BONSAI_B1_ERR_FORMAT;
    const int64_t r = e.shape[0], c = e.shape[1];
    if (r <= 0 || c <= 0 || c % BONSAI_B1_BLOCK_BYTES) return BONSAI_B1_ERR_FORMAT;
    if ((uint64_t)r > (e.end - e.begin) / (uint64_t)c || (uint64_t)r * (uint64_t)c != e.end - e.begin)
        return BONSAI_B1_ERR_FORMAT;
    if (r > INT32_MAX || c / BONSAI_B1_BLOCK_BYTES * BONSAI_B1_BLOCK_SIZE > INT32_MAX) return BONSAI_B1_ERR_FORMAT;
    *rows = r;
    *cols = c;
    return BONSAI_B1_OK;
}

// Pinned host buffers the tensor bytes pass through on their way to the
// device: the mapped file is pageable memory, which the runtime would copy
// through a staging buffer of its own with the host waiting on each piece.
// Here host threads fill one buffer while the DMA engine drains the others.
constexpr size_t kStageMax = 16u << 20; // bytes per buffer
constexpr int kStageBufs = 3;
constexpr size_t kCopySlice = 4u << 20; // bytes per host copy thread

struct Stager {
    void *buf[kStageBufs] = {};
    hipEvent_t ev[kStageBufs] = {};
    size_t bytes = 0;
    int device = -1;

    void release() {
        for (int i = 0; i < kStageBufs; ++i) {
            if (buf[i]) (void)hipHostFree(buf[i]);
            if (ev[i]) (void)hipEventDestroy(ev[i]);
            buf[i] = nullptr;
            ev[i] = nullptr;
        }
        bytes = 0;
        device = -1;
    }
    // Buffers of at least `want` bytes (capped) with events on `dev`.
    bool ensure(size_t want, int dev) {
        want = std::min(kStageMax, (want + 65535) & ~(size_t)65535);
        if (device == dev && bytes >= want) return true;
        release();
        for (int i = 0; i < kStageBufs; ++i) {
            if (hipHostMalloc(&buf[i], want, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&ev[i], hipEventDisableTiming) != hipSuccess) {
                release();
                return false;
            }
        }
        bytes = want;
        device = dev;
        return true;
    }
};

// Host copy of n bytes, split over a few threads for large pieces (one
// thread copying out of the page cache does not keep up with the DMA).
void copy_host(void *dst, const uint8_t *src, size_t n) {
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const size_t parts = std::min<size_t>(std::min<size_t>(4, hw), (n + kCopySlice - 1) / kCopySlice);
    uint8_t *d = static_cast<uint8_t *>(dst);
    const size_t step = parts > 1 ? (n + parts - 1) / parts : n;
    std::vector<std::thread> th;
    try {
        th.reserve(parts);
        for (size_t p = 1; p < parts && p * step < n; ++p) {
            const size_t o = p * step;
            th.emplace_back([=] { memcpy(d + o, src + o, std::min(step, n - o)); });
        }
    } catch (...) {
        // fewer threads than pieces: the pieces without one are copied here
    }
    const size_t rest = std::min(n, step * (th.size() + 1)); // first piece no thread took
    memcpy(d, src, std::min(step, n));
    if (rest < n) memcpy(d + rest, src + rest, n - rest);
    for (auto &t : th) t.join();
}

} // namespace

// An open .safetensors file: the file mapped once and its header parsed
// once, as SafetensorsFile (src/safetensors.h:27-90) holds it.
struct bonsai_b1_safetensors {
    Mapped m;
    uint64_t data_start = 0;
    std::vector<std::pair<std::string, Entry>> entries; // header order
    std::unordered_map<std::string, size_t> by_name;
    Stager stage;
    ~bonsai_b1_safetensors() { stage.release(); }

    int open(const char *path) {
        if (!m.open(path)) return BONSAI_B1_ERR_IO;
        if (m.n < 8) return BONSAI_B1_ERR_FORMAT;
        uint64_t hlen = 0;
        for (int k = 7; k >= 0; --k) hlen = (hlen << 8) | m.p[k];
        if (hlen == 0 || hlen > m.n - 8) return BONSAI_B1_ERR_FORMAT;
        Header h(reinterpret_cast<const char *>(m.p + 8), (size_t)hlen);
        if (!h.index(&entries)) return BONSAI_B1_ERR_FORMAT;
        data_start = 8 + hlen;
        for (size_t i = 0; i < entries.size(); ++i) by_name.emplace(entries[i].first, i);
        return BONSAI_B1_OK;
    }
    // A B1_0 tensor's bytes in the mapping and its dims.
    int find(const char *name, const uint8_t **data, uint64_t *nbytes, int64_t *rows, int64_t *cols) const {
        const auto it = by_name.find(name);
        if (it == by_name.end()) return BONSAI_B1_ERR_NOT_FOUND;
        const Entry &e = entries[it->second].second;
        const int st = b1_check(e, m.n - data_start, rows, cols);
        if (st != BONSAI_B1_OK) return st;
        *data = m.p + data_start + e.begin;
        *nbytes = e.end - e.begin;
        return BONSAI_B1_OK;
    }
};


extern "C" {

int bonsai_b1_safetensors_open(const char *path, bonsai_b1_safetensors **out) {
    if (!path || !out) return BONSAI_B1_ERR_ARG;
    *out = nullptr;
    bonsai_b1_safetensors *f = new (std::nothrow) bonsai_b1_safetensors();
    if (!f) return BONSAI_B1_ERR_IO;
    const int st = f->open(path);
    if (st != BONSAI_B1_OK) {
        delete f;
        return st;
    }
    *out = f;
    return BONSAI_B1_OK;
}

void bonsai_b1_safetensors_close(bonsai_b1_safetensors *f) { delete f; }

int bonsai_b1_safetensors_count(const bonsai_b1_safetensors *f) { return f ? (int)f->entries.size() : -1; }

const char *bonsai_b1_safetensors_name(const bonsai_b1_safetensors *f, int i) {
    if (!f || i < 0 || (size_t)i >= f->entries.size()) return nullptr;
    return f->entries[(size_t)i].first.c_str();
}

int bonsai_b1_safetensors_find(const bonsai_b1_safetensors *f, const char *name, int *in_dim, int *out_dim,
                               uint64_t *data_offset, uint64_t *nbytes) {
    if (!f || !name) return BONSAI_B1_ERR_ARG;
    const uint8_t *data = nullptr;
    uint64_t nb = 0;
    int64_t rows = 0, cols = 0;
    const int st = f->find(name, &data, &nb, &rows, &cols);
    if (st != BONSAI_B1_OK) return st;
    if (in_dim) *in_dim = (int)(cols / BONSAI_B1_BLOCK_BYTES * BONSAI_B1_BLOCK_SIZE);
    if (out_dim) *out_dim = (int)rows;
    if (data_offset) *data_offset = (uint64_t)(data - f->m.p);
    if (nbytes) *nbytes = nb;
    return BONSAI_B1_OK;
}

int bonsai_b1_safetensors_load(bonsai_b1_safetensors *f, const char *const *names, int n, hipStream_t stream,
                               B1Weights *out) {
    if (!f || n < 0 || (n > 0 && (!names || !out))) return BONSAI_B1_ERR_ARG;
    for (int i = 0; i < n; ++i) out[i] = B1Weights{};
    if (n == 0) return BONSAI_B1_OK;
    // Every name is resolved before anything is allocated.
    struct Job {
        const uint8_t *src;
        uint64_t nb;
        int in_dim, out_dim;
    };
    std::vector<Job> jobs((size_t)n);
    uint64_t largest = 0;
    for (int i = 0; i < n; ++i) {
        if (!names[i]) return BONSAI_B1_ERR_ARG;
        int64_t rows = 0, cols = 0;
        const int st = f->find(names[i], &jobs[(size_t)i].src, &jobs[(size_t)i].nb, &rows, &cols);
        if (st != BONSAI_B1_OK) return st;
        jobs[(size_t)i].in_dim = (int)(cols / BONSAI_B1_BLOCK_BYTES * BONSAI_B1_BLOCK_SIZE);
        jobs[(size_t)i].out_dim = (int)rows;
        largest = std::max(largest, jobs[(size_t)i].nb);
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return BONSAI_B1_ERR_DEVICE;
    if (!f->stage.ensure((size_t)largest, dev)) return BONSAI_B1_ERR_HIP;
    int status = BONSAI_B1_OK;
    for (int i = 0; i < n && status == BONSAI_B1_OK; ++i) {
        void *d = nullptr;
        if (hipMalloc(&d, (size_t)jobs[(size_t)i].nb) != hipSuccess) {
            status = BONSAI_B1_ERR_HIP;
            break;
        }
        out[i] = B1Weights{d, jobs[(size_t)i].in_dim, jobs[(size_t)i].out_dim, (size_t)jobs[(size_t)i].nb, dev};
    }
    // Chunks go round the staging buffers: a buffer is refilled once the
    // copy that last read it has completed.
    Stager &sg = f->stage;
    bool pending[kStageBufs] = {};
    int slot = 0;
    for (int i = 0; i < n && status == BONSAI_B1_OK; ++i) {
        const Job &j = jobs[(size_t)i];
        uint8_t *dst = static_cast<uint8_t *>(out[i].data);
        for (uint64_t off = 0; off < j.nb; off += sg.bytes) {
            const size_t len = (size_t)std::min<uint64_t>(sg.bytes, j.nb - off);
            if (pending[slot] && hipEventSynchronize(sg.ev[slot]) != hipSuccess) {
                status = BONSAI_B1_ERR_HIP;
                break;
            }
            copy_host(sg.buf[slot], j.src + off, len);
            if (hipMemcpyAsync(dst + off, sg.buf[slot], len, hipMemcpyHostToDevice, stream) != hipSuccess ||
                hipEventRecord(sg.ev[slot], stream) != hipSuccess) {
                status = BONSAI_B1_ERR_HIP;
                break;
            }
            pending[slot] = true;
            slot = (slot + 1) % kStageBufs;
        }
    }
    // The staging buffers are free, and the weights resident, once the
    // stream has passed the last copy.
    if (hipStreamSynchronize(stream) != hipSuccess && status == BONSAI_B1_OK) status = BONSAI_B1_ERR_HIP;
    if (status != BONSAI_B1_OK) {
        for (int i = 0; i < n; ++i) {
            (void)bonsai_b1_weights_free(&out[i]);
            out[i] = B1Weights{};
        }
    }
    return status;
}

int bonsai_b1_safetensors_info(const char *path, const char *name, int *in_dim, int *out_dim,
                               uint64_t *data_offset, uint64_t *nbytes) {
    if (!path || !name) return BONSAI_B1_ERR_ARG;
    bonsai_b1_safetensors f;
    const int st = f.open(path);
    if (st != BONSAI_B1_OK) return st;
    return bonsai_b1_safetensors_find(&f, name, in_dim, out_dim, data_offset, nbytes);
}

int bonsai_b1_weights_load_safetensors(const char *path, const char *name, hipStream_t stream, B1Weights *out) {
    if (!path || !name || !out) return BONSAI_B1_ERR_ARG;
    bonsai_b1_safetensors f;
    const int st = f.open(path);
    if (st != BONSAI_B1_OK) return st;
    return bonsai_b1_safetensors_load(&f, &name, 1, stream, out);
}

} // extern "C"
