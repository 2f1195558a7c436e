/*
 * tmt_moe_ckpt.hpp -- the MoE block's parameters in TMT's V3 checkpoint byte
 * layout (C++17, POSIX, host side over tmt_moe.h).
 *
 * Byte layout (all integers little-endian u64, floats IEEE fp32):
 *
 *   offset 0   magic 0x33544b5043544d54 (the ASCII bytes "TMTCPKT3")
 *   offset 8   L, the length of the configuration text, 1 <= L <= 16384
 *   offset 16  L bytes of "key=value\n" lines
 *              then P, the number of parameter records
 *              then P records, each: n, n master values, n first moments,
 *              n second moments (12n + 8 bytes)
 *   last 8     FNV-1a-64 (offset basis 0xcbf29ce484222325, prime
 *              0x100000001b3) of every byte before it
 *
 * The record format and the trailer are TMT's (tmt-cuda/src/checkpoint.h:
 * records :143-150, trailer :46-73, magic :75); the bf16 work copy of each
 * parameter is not stored and is regenerated from the master on load
 * (checkpoint.h:149). Parameters follow the model's registration order
 * (tmt-cuda/src/model.cu:222-246), see moe_layer_param_sizes. A model-level
 * writer can embed a layer's records unchanged with write_records.
 *
 * A block file carries the keys "dim", "experts", "topk" and, where they
 * apply, "moe_hidden" (up/down experts; TMT has no key for that shape) and
 * "moe_layernorm". Architecture checks compare the whole text.
 *
 * Implementation: the writer appends through one POSIX descriptor while
 * hashing, then appends the trailer, fsyncs the file, renames it over the
 * destination and fsyncs the directory, so a crash leaves either the old or
 * the complete new file. The reader maps the whole file read-only, checks
 * size and trailer before anything is parsed, then walks the mapping with a
 * bounds-checked cursor and copies records straight from it to the device.
 * Errors throw std::runtime_error with a "tmt_ckpt:" prefix.
 */
#pragma once

#include <hip/hip_runtime_api.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "tmt_moe.h"

namespace tmt_ckpt {

constexpr uint64_t kFnvOffset = 0xcbf29ce484222325ull;
constexpr uint64_t kFnvPrime = 0x100000001b3ull;
constexpr uint64_t kMagic = 0x33544b5043544d54ull;  // "TMTCPKT3" read as a little-endian u64
constexpr uint64_t kMaxConfigText = 16384;

// FNV-1a-64 of n bytes, continuing from `state` (kFnvOffset starts a hash).
inline uint64_t fnv1a64(const void* p, size_t n, uint64_t state = kFnvOffset) {
    const unsigned char* c = static_cast<const unsigned char*>(p);
    const unsigned char* end = c + n;
    while (c != end) {
        state ^= *c++;
        state *= kFnvPrime;
    }
    return state;
}

[[noreturn]] inline void raise(const std::string& what) { throw std::runtime_error("tmt_ckpt: " + what); }

inline void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) raise(std::string(what) + ": " + hipGetErrorString(e));
}

// ------------------------------------------------------------- layer shape --

// One parameter's device state (the reference's Par, tmt-cuda/src/train.cu:35-41).
struct Param {
    float* master = nullptr;
    float* m = nullptr;
    float* v = nullptr;
    uint16_t* work = nullptr;  // bf16 copy used by the kernels, or nullptr
    int64_t n = 0;
};

struct LayerShape {
    int dim = 0, experts = 0, topk = 0, hidden = 0;
    bool layernorm = false;  // gamma and beta are registered before the router (model.cu:222-231)
};

// Element counts of the layer's parameters in registration order:
// [gamma, beta,] router [E][D], then per expert W_e [D][D] (hidden == 0) or
// W_up[e] [h][D] followed by W_down[e] [D][h].
inline std::vector<int64_t> moe_layer_param_sizes(const LayerShape& s) {
    const int64_t D = s.dim, H = s.hidden;
    std::vector<int64_t> sizes;
    if (s.layernorm) sizes.insert(sizes.end(), {D, D});
    sizes.push_back(D * s.experts);
    for (int e = 0; e < s.experts; ++e) {
        if (H == 0) {
            sizes.push_back(D * D);
        } else {
            sizes.push_back(H * D);
            sizes.push_back(D * H);
        }
    }
    return sizes;
}

inline std::string layer_config_text(const LayerShape& s) {
    std::string t = "dim=" + std::to_string(s.dim) + "\nexperts=" + std::to_string(s.experts) +
                    "\ntopk=" + std::to_string(s.topk) + "\n";
    if (s.hidden > 0) t += "moe_hidden=" + std::to_string(s.hidden) + "\n";
    if (s.layernorm) t += "moe_layernorm=1\n";
    return t;
}

inline void check_params(const LayerShape& s, const std::vector<Param>& ps) {
    const std::vector<int64_t> want = moe_layer_param_sizes(s);
    if (want.size() != ps.size())
        raise("the layer has " + std::to_string(want.size()) + " parameters, " + std::to_string(ps.size()) +
              " were passed");
    for (size_t i = 0; i < want.size(); ++i)
        if (ps[i].n != want[i])
            raise("parameter " + std::to_string(i) + " has " + std::to_string(ps[i].n) +
                  " elements, the layer shape gives " + std::to_string(want[i]));
}

// ------------------------------------------------------------------ writer --

// Append-only writer: every byte goes to one descriptor and into the running
// hash. commit() appends the trailer and makes the file durable under its
// final name; a Writer destroyed without commit() removes its partial file.
class Writer {
public:
    explicit Writer(const std::string& path)
        : final_(path), partial_(path + ".partial." + std::to_string(::getpid())) {
        fd_ = ::open(partial_.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
        if (fd_ < 0) raise("cannot create " + partial_ + ": " + std::strerror(errno));
    }
    ~Writer() {
        if (fd_ >= 0) ::close(fd_);
        if (!committed_) ::unlink(partial_.c_str());
    }
    Writer(const Writer&) = delete;
    Writer& operator=(const Writer&) = delete;

    void put(const void* p, size_t n) {
        hash_ = fnv1a64(p, n, hash_);
        emit(p, n);
    }
    void put_u64(uint64_t v) { put(&v, sizeof v); }
    // Device bytes, staged through host memory in 4 MiB pieces.
    void put_device(const void* dev, size_t n) {
        constexpr size_t kPiece = size_t(4) << 20;
        if (stage_.size() < kPiece) stage_.resize(kPiece);
        const char* src = static_cast<const char*>(dev);
        for (size_t done = 0; done < n;) {
            const size_t k = n - done < kPiece ? n - done : kPiece;
            hip_ok(hipMemcpy(stage_.data(), src + done, k, hipMemcpyDeviceToHost), "reading device memory");
            put(stage_.data(), k);
            done += k;
        }
    }
    uint64_t hash() const { return hash_; }

    void commit() {
        const uint64_t trailer = hash_;
        emit(&trailer, sizeof trailer);
        if (::fsync(fd_) != 0) raise("fsync of " + partial_ + " failed: " + std::strerror(errno));
        const int rc = ::close(fd_);
        fd_ = -1;
        if (rc != 0) raise("closing " + partial_ + " failed: " + std::strerror(errno));
        if (::rename(partial_.c_str(), final_.c_str()) != 0)
            raise("cannot move " + partial_ + " to " + final_ + ": " + std::strerror(errno));
        committed_ = true;
        // make the rename itself durable
        const size_t slash = final_.find_last_of('/');
        const std::string dir = slash == std::string::npos ? "." : (slash == 0 ? "/" : final_.substr(0, slash));
        const int dfd = ::open(dir.c_str(), O_RDONLY | O_DIRECTORY | O_CLOEXEC);
        if (dfd >= 0) {
            (void)::fsync(dfd);
            ::close(dfd);
        }
    }

private:
    void emit(const void* p, size_t n) {
        const char* c = static_cast<const char*>(p);
        while (n > 0) {
            const ssize_t w = ::write(fd_, c, n);
            if (w < 0 && errno == EINTR) continue;
            if (w <= 0) raise("writing " + partial_ + " failed: " + std::strerror(errno));
            c += w;
            n -= (size_t)w;
        }
    }
    std::string final_, partial_;
    int fd_ = -1;
    bool committed_ = false;
    uint64_t hash_ = kFnvOffset;
    std::vector<char> stage_;
};

// ------------------------------------------------------------------ reader --

// Read-only mapping of a whole checkpoint file whose trailer has been
// checked: the constructor throws for files shorter than magic + trailer or
// whose last 8 bytes differ from the hash of the rest.
class FileImage {
public:
    explicit FileImage(const std::string& path) : path_(path) {
        const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) raise("cannot open " + path + ": " + std::strerror(errno));
        struct stat st;
        if (::fstat(fd, &st) != 0) {
            ::close(fd);
            raise("cannot stat " + path);
        }
        size_ = (size_t)st.st_size;
        if (size_ < 16) {
            ::close(fd);
            raise(path + " has " + std::to_string(size_) + " bytes, fewer than magic + trailer");
        }
        void* m = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        if (m == MAP_FAILED) raise("cannot map " + path + ": " + std::strerror(errno));
        base_ = static_cast<const unsigned char*>(m);
        uint64_t stored;
        std::memcpy(&stored, base_ + size_ - 8, 8);
        const uint64_t actual = fnv1a64(base_, size_ - 8);
        if (stored != actual) {
            ::munmap(const_cast<unsigned char*>(base_), size_);
            base_ = nullptr;
            char msg[128];
            std::snprintf(msg, sizeof msg, " is corrupt: trailer %016llx, content hashes to %016llx",
                          (unsigned long long)stored, (unsigned long long)actual);
            raise(path + msg);
        }
    }
    ~FileImage() {
        if (base_) ::munmap(const_cast<unsigned char*>(base_), size_);
    }
    FileImage(const FileImage&) = delete;
    FileImage& operator=(const FileImage&) = delete;
    const unsigned char* data() const { return base_; }
    size_t payload_size() const { return size_ - 8; }  // bytes before the trailer
    const std::string& path() const { return path_; }

private:
    std::string path_;
    const unsigned char* base_ = nullptr;
    size_t size_ = 0;
};

// Bounds-checked walk over a FileImage's payload.
class Cursor {
public:
    explicit Cursor(const FileImage& f) : img_(f), at_(0), end_(f.payload_size()) {}
    const unsigned char* take(size_t n, const char* what) {
        if (n > end_ - at_)
            raise(img_.path() + ": " + what + " needs " + std::to_string(n) + " bytes at offset " +
                  std::to_string(at_) + ", the payload ends at " + std::to_string(end_));
        const unsigned char* p = img_.data() + at_;
        at_ += n;
        return p;
    }
    uint64_t u64(const char* what) {
        uint64_t v;
        std::memcpy(&v, take(8, what), 8);
        return v;
    }
    bool at_end() const { return at_ == end_; }
    size_t offset() const { return at_; }
    const std::string& path() const { return img_.path(); }

private:
    const FileImage& img_;
    size_t at_, end_;
};

// Throws unless `path` is a complete checkpoint (size and trailer).
inline void check_file(const std::string& path) { FileImage img(path); }

// ----------------------------------------------------------------- records --

// P, then per parameter: n, master, m, v.
inline void write_records(Writer& w, const std::vector<Param>& ps) {
    w.put_u64(ps.size());
    for (const Param& p : ps) {
        const uint64_t n = (uint64_t)p.n;
        w.put_u64(n);
        w.put_device(p.master, n * 4);
        w.put_device(p.m, n * 4);
        w.put_device(p.v, n * 4);
    }
}

// Reads the records into `ps` (counts and sizes must match) and regenerates
// the bf16 work copies from the masters on `stream`.
inline void read_records(Cursor& c, std::vector<Param>& ps, hipStream_t stream = nullptr) {
    const uint64_t count = c.u64("record count");
    if (count != ps.size())
        raise(c.path() + " holds " + std::to_string(count) + " records, " + std::to_string(ps.size()) +
              " parameters were passed");
    for (size_t i = 0; i < ps.size(); ++i) {
        Param& p = ps[i];
        const uint64_t n = c.u64("record length");
        if (n != (uint64_t)p.n)
            raise(c.path() + ": record " + std::to_string(i) + " has " + std::to_string(n) +
                  " values, the parameter has " + std::to_string(p.n));
        float* dst[3] = {p.master, p.m, p.v};
        for (float* d : dst) hip_ok(hipMemcpy(d, c.take(n * 4, "record values"), n * 4, hipMemcpyHostToDevice),
                                    "writing device memory");
        if (p.work && tmt_moe_f32_to_bf16(stream, p.master, p.work, (int64_t)n) != TMT_MOE_OK)
            raise(std::string("bf16 work copy: ") + tmt_moe_last_error());
    }
    hip_ok(hipStreamSynchronize(stream), "bf16 work copy");
}

// --------------------------------------------------------------- block file --

inline void save_layer(const std::string& path, const LayerShape& s, const std::vector<Param>& ps) {
    check_params(s, ps);
    const std::string text = layer_config_text(s);
    Writer w(path);
    w.put_u64(kMagic);
    w.put_u64(text.size());
    w.put(text.data(), text.size());
    write_records(w, ps);
    w.commit();
}

// The whole file is checked before any parameter is written; a file of
// another layer shape is refused.
inline void load_layer(const std::string& path, const LayerShape& s, std::vector<Param>& ps,
                       hipStream_t stream = nullptr) {
    check_params(s, ps);
    FileImage img(path);
    Cursor c(img);
    if (c.u64("magic") != kMagic) raise(path + " is not a V3 checkpoint (magic differs)");
    const uint64_t len = c.u64("configuration length");
    if (len == 0 || len > kMaxConfigText)
        raise(path + ": configuration text of " + std::to_string(len) + " bytes is outside [1, 16384]");
    const std::string stored(reinterpret_cast<const char*>(c.take(len, "configuration text")), len);
    const std::string want = layer_config_text(s);
    if (stored != want) raise(path + " stores the layer\n" + stored + "but this layer is\n" + want);
    // Shape the records before touching the device: count and lengths must
    // cover the payload exactly.
    {
        Cursor probe = c;
        if (probe.u64("record count") != ps.size()) raise(path + ": record count differs from the layer");
        for (const Param& p : ps) {
            if (probe.u64("record length") != (uint64_t)p.n) raise(path + ": a record length differs from the layer");
            probe.take((size_t)p.n * 12, "record values");
        }
        if (!probe.at_end())
            raise(path + ": " + std::to_string(img.payload_size() - probe.offset()) + " unexpected bytes after the records");
    }
    read_records(c, ps, stream);
}

}  // namespace tmt_ckpt
