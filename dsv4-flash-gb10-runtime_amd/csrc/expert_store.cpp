// expert_store.cpp — safetensors snapshot reader that fills the HBM-resident
// expert tensors of the routed MoE path (host code; C ABI in
// include/dsv4_expert_store.h).
//
// A safetensors file is an 8-byte little-endian header length H, H bytes of
// JSON ({name: {"dtype", "shape", "data_offsets": [begin, end]}, optional
// "__metadata__"}), then the tensor bytes at 8 + H + begin. A sharded
// snapshot adds model.safetensors.index.json ({"weight_map": {name: shard}}).
// Every header is parsed once at open; reads are pread() on file descriptors
// kept open for the store's lifetime. Device loads stage through two pinned
// buffers so that the next read overlaps the previous host-to-device copy.

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include <hip/hip_runtime.h>

#include "dsv4_expert_store.h"

namespace {

// ------------------------------------------------------------------ JSON --

struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    bool is_int = false;
    int64_t inum = 0;
    double num = 0.0;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;

    const JVal* get(const char* key) const {
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

// Recursive-descent parser for RFC 8259 JSON (depth-limited).
class JParser {
  public:
    JParser(const char* p, size_t n) : p_(p), end_(p + n) {}

    bool parse(JVal& out) {
        ws();
        if (!value(out, 0)) return false;
        ws();
        return p_ == end_;
    }

  private:
    const char* p_;
    const char* end_;

    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }
    bool lit(const char* s) {
        const size_t n = std::strlen(s);
        if ((size_t)(end_ - p_) < n || std::memcmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    bool value(JVal& v, int depth) {
        if (depth > 64 || p_ >= end_) return false;
        switch (*p_) {
            case '{': return object(v, depth);
            case '[': return array(v, depth);
            case '"': v.kind = JVal::Str; return string(v.str);
            case 't': v.kind = JVal::Bool; v.b = true; return lit("true");
            case 'f': v.kind = JVal::Bool; v.b = false; return lit("false");
            case 'n': v.kind = JVal::Null; return lit("null");
            default: return number(v);
        }
    }
    bool object(JVal& v, int depth) {
        v.kind = JVal::Obj;
        ++p_;
        ws();
        if (p_ < end_ && *p_ == '}') { ++p_; return true; }
        while (true) {
            ws();
            std::string key;
            if (p_ >= end_ || *p_ != '"' || !string(key)) return false;
            ws();
            if (p_ >= end_ || *p_ != ':') return false;
            ++p_;
            ws();
            JVal x;
            if (!value(x, depth + 1)) return false;
            v.obj.emplace_back(std::move(key), std::move(x));
            ws();
            if (p_ >= end_) return false;
            if (*p_ == ',') { ++p_; continue; }
            if (*p_ == '}') { ++p_; return true; }
            return false;
        }
    }
    bool array(JVal& v, int depth) {
        v.kind = JVal::Arr;
        ++p_;
        ws();
        if (p_ < end_ && *p_ == ']') { ++p_; return true; }
        while (true) {
            ws();
            JVal x;
            if (!value(x, depth + 1)) return false;
            v.arr.push_back(std::move(x));
            ws();
            if (p_ >= end_) return false;
            if (*p_ == ',') { ++p_; continue; }
            if (*p_ == ']') { ++p_; return true; }
            return false;
        }
    }
    static void utf8(std::string& s, uint32_t cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t& out) {
        if (end_ - p_ < 4) return false;
        out = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            out <<= 4;
            if (c >= '0' && c <= '9') out |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') out |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') out |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string& s) {
        ++p_;  // opening quote
        while (p_ < end_) {
            const char c = *p_++;
            if (c == '"') return true;
            if ((unsigned char)c < 0x20) return false;
            if (c != '\\') { s += c; continue; }
            if (p_ >= end_) return false;
            const char e = *p_++;
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
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                        uint32_t lo;
                        if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return false;
                        p_ += 2;
                        if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return false;
                    }
                    utf8(s, cp);
                    break;
                }
                default: return false;
            }
        }
        return false;
    }
    bool number(JVal& v) {
        const char* start = p_;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
        if (*p_ == '0') ++p_;
        else while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        bool integral = true;
        if (p_ < end_ && *p_ == '.') {
            integral = false;
            ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integral = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        const std::string text(start, p_);
        v.kind = JVal::Num;
        v.num = std::strtod(text.c_str(), nullptr);
        if (integral) {
            errno = 0;
            v.inum = std::strtoll(text.c_str(), nullptr, 10);
            v.is_int = errno == 0;
        }
        return true;
    }
};

// ----------------------------------------------------------------- files --

bool read_full(int fd, void* dst, int64_t n, int64_t off) {
    uint8_t* p = static_cast<uint8_t*>(dst);
    while (n > 0) {
        const ssize_t r = ::pread(fd, p, (size_t)n, (off_t)off);
        if (r < 0) {
            if (errno == EINTR) continue;
            return false;
        }
        if (r == 0) return false;  // past the end of the file
        p += r;
        n -= r;
        off += r;
    }
    return true;
}

bool read_file(const std::string& path, std::string& out) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return false;
    struct stat st;
    bool ok = ::fstat(fd, &st) == 0 && st.st_size < ((int64_t)1 << 31);
    if (ok) {
        out.resize((size_t)st.st_size);
        ok = read_full(fd, &out[0], st.st_size, 0);
    }
    ::close(fd);
    return ok;
}

int64_t dtype_size(const std::string& d) {
    if (d == "I8" || d == "U8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2" || d == "F8_E8M0") return 1;
    if (d == "I16" || d == "U16" || d == "F16" || d == "BF16") return 2;
    if (d == "I32" || d == "U32" || d == "F32") return 4;
    if (d == "I64" || d == "U64" || d == "F64") return 8;
    return 0;  // unknown: the byte range is taken as given
}

struct Tensor {
    int shard;
    std::string dtype;
    std::vector<int64_t> shape;
    int64_t offset;  // absolute file offset
    int64_t nbytes;
};

struct Shard {
    std::string path;
    int fd;
};

bool is_dir(const std::string& p) {
    struct stat st;
    return ::stat(p.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
}

bool is_file(const std::string& p) {
    struct stat st;
    return ::stat(p.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

// Pinned staging buffers and their reuse events, freed on scope exit.
struct Staging {
    void* buf[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool used[2] = {false, false};
    ~Staging() {
        for (int i = 0; i < 2; ++i) {
            if (ev[i]) {
                if (used[i]) (void)hipEventSynchronize(ev[i]);
                (void)hipEventDestroy(ev[i]);
            }
            if (buf[i]) (void)hipHostFree(buf[i]);
        }
    }
    hipError_t init(size_t bytes) {
        for (int i = 0; i < 2; ++i) {
            hipError_t e = hipHostMalloc(&buf[i], bytes, hipHostMallocDefault);
            if (e != hipSuccess) return e;
            e = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    // Buffer i may be refilled once its previous copy is complete.
    hipError_t acquire(int i) {
        if (!used[i]) return hipSuccess;
        used[i] = false;
        return hipEventSynchronize(ev[i]);
    }
    hipError_t release(int i, hipStream_t s) {
        used[i] = true;
        return hipEventRecord(ev[i], s);
    }
    hipError_t finish() {
        for (int i = 0; i < 2; ++i) {
            const hipError_t e = acquire(i);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
};

}  // namespace

struct dsv4_store {
    std::vector<Shard> shards;
    std::unordered_map<std::string, Tensor> tensors;

    ~dsv4_store() {
        for (auto& s : shards)
            if (s.fd >= 0) ::close(s.fd);
    }

    // Opens one shard and indexes its tensors.
    bool add_shard(const std::string& path) {
        const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) {
            std::fprintf(stderr, "dsv4_store: cannot open %s: %s\n", path.c_str(), std::strerror(errno));
            return false;
        }
        shards.push_back(Shard{path, fd});
        const int si = (int)shards.size() - 1;
        struct stat st;
        if (::fstat(fd, &st) != 0) return false;
        const int64_t fsize = st.st_size;
        uint8_t lenb[8];
        if (fsize < 8 || !read_full(fd, lenb, 8, 0)) {
            std::fprintf(stderr, "dsv4_store: %s: too short for a safetensors header\n", path.c_str());
            return false;
        }
        uint64_t hlen = 0;
        for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | lenb[i];
        if (hlen > ((uint64_t)1 << 30) || (int64_t)(8 + hlen) > fsize) {
            std::fprintf(stderr, "dsv4_store: %s: bad header length %llu\n", path.c_str(),
                         (unsigned long long)hlen);
            return false;
        }
        std::string hdr((size_t)hlen, '\0');
        if (!read_full(fd, &hdr[0], (int64_t)hlen, 8)) return false;
        JVal root;
        if (!JParser(hdr.data(), hdr.size()).parse(root) || root.kind != JVal::Obj) {
            std::fprintf(stderr, "dsv4_store: %s: header is not a JSON object\n", path.c_str());
            return false;
        }
        const int64_t data0 = 8 + (int64_t)hlen;
        for (const auto& kv : root.obj) {
            if (kv.first == "__metadata__") continue;
            const JVal& t = kv.second;
            const JVal* dt = t.get("dtype");
            const JVal* sh = t.get("shape");
            const JVal* off = t.get("data_offsets");
            bool ok = t.kind == JVal::Obj && dt && dt->kind == JVal::Str && sh && sh->kind == JVal::Arr &&
                      off && off->kind == JVal::Arr && off->arr.size() == 2 && dt->str.size() < 16;
            Tensor rec{si, ok ? dt->str : std::string(), {}, 0, 0};
            int64_t count = 1;
            if (ok) {
                for (const JVal& d : sh->arr) {
                    ok = ok && d.kind == JVal::Num && d.is_int && d.inum >= 0;
                    if (!ok) break;
                    rec.shape.push_back(d.inum);
                    count *= d.inum;
                }
            }
            if (ok) {
                const JVal& b = off->arr[0];
                const JVal& e = off->arr[1];
                ok = b.kind == JVal::Num && b.is_int && e.kind == JVal::Num && e.is_int && b.inum >= 0 &&
                     e.inum >= b.inum && data0 + e.inum <= fsize;
                if (ok) {
                    rec.offset = data0 + b.inum;
                    rec.nbytes = e.inum - b.inum;
                }
            }
            const int64_t es = ok ? dtype_size(rec.dtype) : 0;
            if (ok && es > 0) ok = rec.nbytes == count * es;
            if (!ok) {
                std::fprintf(stderr, "dsv4_store: %s: bad entry for tensor %s\n", path.c_str(), kv.first.c_str());
                return false;
            }
            if (!tensors.emplace(kv.first, std::move(rec)).second) {
                std::fprintf(stderr, "dsv4_store: tensor %s appears twice\n", kv.first.c_str());
                return false;
            }
        }
        return true;
    }

    const Tensor* find(const char* name) const {
        const auto it = tensors.find(name);
        return it == tensors.end() ? nullptr : &it->second;
    }

    bool read(const Tensor& t, void* dst, int64_t n, int64_t at) const {
        return read_full(shards[t.shard].fd, dst, n, t.offset + at);
    }
};

namespace {

bool open_snapshot(dsv4_store& s, const std::string& path) {
    if (is_file(path)) return s.add_shard(path);
    if (!is_dir(path)) {
        std::fprintf(stderr, "dsv4_store: %s is neither a file nor a directory\n", path.c_str());
        return false;
    }
    const std::string index = path + "/model.safetensors.index.json";
    if (!is_file(index)) {
        const std::string single = path + "/model.safetensors";
        if (is_file(single)) return s.add_shard(single);
        std::fprintf(stderr, "dsv4_store: %s has no model.safetensors.index.json\n", path.c_str());
        return false;
    }
    std::string text;
    JVal root;
    if (!read_file(index, text) || !JParser(text.data(), text.size()).parse(root) || root.kind != JVal::Obj) {
        std::fprintf(stderr, "dsv4_store: cannot parse %s\n", index.c_str());
        return false;
    }
    const JVal* wm = root.get("weight_map");
    if (!wm || wm->kind != JVal::Obj) {
        std::fprintf(stderr, "dsv4_store: %s has no weight_map object\n", index.c_str());
        return false;
    }
    std::vector<std::string> files;
    for (const auto& kv : wm->obj) {
        if (kv.second.kind != JVal::Str || kv.second.str.empty() || kv.second.str.find('/') != std::string::npos) {
            std::fprintf(stderr, "dsv4_store: bad shard name for %s\n", kv.first.c_str());
            return false;
        }
        bool seen = false;
        for (const auto& f : files) seen = seen || f == kv.second.str;
        if (!seen) files.push_back(kv.second.str);
    }
    for (const auto& f : files)
        if (!s.add_shard(path + "/" + f)) return false;
    // Every name of the weight map lives in the shard it names.
    for (const auto& kv : wm->obj) {
        const Tensor* t = s.find(kv.first.c_str());
        if (!t || s.shards[t->shard].path != path + "/" + kv.second.str) {
            std::fprintf(stderr, "dsv4_store: %s is not in %s\n", kv.first.c_str(), kv.second.str.c_str());
            return false;
        }
    }
    return true;
}

constexpr int64_t kChunk = 64 << 20;  // staging chunk of dsv4_store_load_tensor

}  // namespace

extern "C" dsv4_store* dsv4_store_open(const char* path) {
    if (path == nullptr) return nullptr;
    dsv4_store* s = new dsv4_store();
    if (!open_snapshot(*s, path)) {
        delete s;
        return nullptr;
    }
    return s;
}

extern "C" int dsv4_store_close(dsv4_store* store) {
    delete store;
    return 0;
}

extern "C" int dsv4_store_count(const dsv4_store* store) {
    return store ? (int)store->tensors.size() : -2;
}

extern "C" int dsv4_store_tensor_info(const dsv4_store* store, const char* name, char dtype[16],
                                      int64_t shape[8], int* ndim, int64_t* nbytes) {
    if (!store || !name || !dtype || !shape || !ndim || !nbytes) return -2;
    const Tensor* t = store->find(name);
    if (!t) return -1;
    if (t->shape.size() > 8) return -3;
    std::snprintf(dtype, 16, "%s", t->dtype.c_str());
    for (size_t i = 0; i < t->shape.size(); ++i) shape[i] = t->shape[i];
    *ndim = (int)t->shape.size();
    *nbytes = t->nbytes;
    return 0;
}

extern "C" int dsv4_store_read(const dsv4_store* store, const char* name, void* dst, int64_t capacity) {
    if (!store || !name || (!dst && capacity > 0)) return -2;
    const Tensor* t = store->find(name);
    if (!t) return -1;
    if (capacity < t->nbytes) return -3;
    return store->read(*t, dst, t->nbytes, 0) ? 0 : -5;
}

extern "C" int dsv4_store_load_tensor(dsv4_store* store, const char* name, void* dst_dev, int64_t capacity,
                                      hipStream_t stream) {
    if (!store || !name || !dst_dev) return -2;
    const Tensor* t = store->find(name);
    if (!t) return -1;
    if (capacity < t->nbytes) return -3;
    if (t->nbytes == 0) return 0;
    Staging st;
    const int64_t chunk = t->nbytes < kChunk ? t->nbytes : kChunk;
    if (st.init((size_t)chunk) != hipSuccess) return -6;
    int i = 0;
    for (int64_t at = 0; at < t->nbytes; at += chunk, i ^= 1) {
        const int64_t n = t->nbytes - at < chunk ? t->nbytes - at : chunk;
        if (st.acquire(i) != hipSuccess) return -6;
        if (!store->read(*t, st.buf[i], n, at)) return -5;
        if (hipMemcpyAsync(static_cast<uint8_t*>(dst_dev) + at, st.buf[i], (size_t)n, hipMemcpyHostToDevice,
                           stream) != hipSuccess ||
            st.release(i, stream) != hipSuccess)
            return -6;
    }
    return st.finish() == hipSuccess ? 0 : -6;
}

extern "C" int dsv4_store_load_experts(dsv4_store* store, int layer, const char* proj, int n_experts,
                                       void* packed_dev, int64_t packed_expert_stride, void* scale_dev,
                                       int64_t scale_expert_stride, int64_t* rows, int64_t* cols,
                                       hipStream_t stream) {
    if (!store || !proj || !packed_dev || !scale_dev || n_experts < 1 || layer < 0) return -2;
    if (std::strcmp(proj, "w1") != 0 && std::strcmp(proj, "w2") != 0 && std::strcmp(proj, "w3") != 0) return -2;
    // Resolve and check every expert before the first copy.
    std::vector<const Tensor*> wt((size_t)n_experts), sc((size_t)n_experts);
    int64_t R = -1, C = -1;
    for (int e = 0; e < n_experts; ++e) {
        const std::string base = "layers." + std::to_string(layer) + ".ffn.experts." + std::to_string(e) + "." + proj;
        wt[e] = store->find((base + ".weight").c_str());
        sc[e] = store->find((base + ".scale").c_str());
        if (!wt[e] || !sc[e]) {
            std::fprintf(stderr, "dsv4_store: %s.weight or .scale missing\n", base.c_str());
            return -1;
        }
        const Tensor& w = *wt[e];
        const Tensor& s = *sc[e];
        const bool shapes = w.dtype == "I8" && s.dtype == "F8_E8M0" && w.shape.size() == 2 && s.shape.size() == 2 &&
                            w.shape[0] == s.shape[0] && s.shape[1] * 16 == w.shape[1] && w.shape[1] > 0;
        if (!shapes || (e > 0 && (w.shape[0] != R || 2 * w.shape[1] != C))) {
            std::fprintf(stderr, "dsv4_store: %s: want I8 [rows, cols/2] + F8_E8M0 [rows, cols/32], the same for every expert\n",
                         base.c_str());
            return -4;
        }
        R = w.shape[0];
        C = 2 * w.shape[1];
    }
    const int64_t wbytes = wt[0]->nbytes;
    const int64_t sbytes = sc[0]->nbytes;
    if (packed_expert_stride < wbytes || scale_expert_stride < sbytes) return -3;
    if (rows) *rows = R;
    if (cols) *cols = C;
    Staging st;
    if (st.init((size_t)(wbytes + sbytes)) != hipSuccess) return -6;
    for (int e = 0; e < n_experts; ++e) {
        const int i = e & 1;
        if (st.acquire(i) != hipSuccess) return -6;
        uint8_t* buf = static_cast<uint8_t*>(st.buf[i]);
        if (!store->read(*wt[e], buf, wbytes, 0) || !store->read(*sc[e], buf + wbytes, sbytes, 0)) return -5;
        if (hipMemcpyAsync(static_cast<uint8_t*>(packed_dev) + (int64_t)e * packed_expert_stride, buf,
                           (size_t)wbytes, hipMemcpyHostToDevice, stream) != hipSuccess ||
            hipMemcpyAsync(static_cast<uint8_t*>(scale_dev) + (int64_t)e * scale_expert_stride, buf + wbytes,
                           (size_t)sbytes, hipMemcpyHostToDevice, stream) != hipSuccess ||
            st.release(i, stream) != hipSuccess)
            return -6;
    }
    return st.finish() == hipSuccess ? 0 : -6;
}
