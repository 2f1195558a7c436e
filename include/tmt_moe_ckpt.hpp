/*
 * tmt_moe_ckpt.hpp -- the MoE block's parameters in the reference's V3
 * checkpoint layout (C++17, host side, over tmt_moe.h).
 *
 * The reference writes every parameter of the model as one record, in the
 * order the parameters were registered (tmt-cuda/src/checkpoint.h:143-150;
 * registration order of a layer tmt-cuda/src/model.cu:222-246):
 *   u64 n, then n fp32 master weights, n fp32 first moments, n fp32 second
 *   moments; the bf16 work copy is regenerated from the master on load.
 * The whole file is covered by a 64-bit FNV-1a hash written as an 8-byte
 * trailer (checkpoint.h:11-16, 46-57, 59-73); a reader rejects a file whose
 * trailer does not match or that has bytes after it.
 *
 * This header keeps those records byte for byte, so a model-level writer
 * embeds a layer's records unchanged, and gives the block a file of its own
 * with the same framing:
 *   u64 magic "TMTCPKT3" (checkpoint.h:75), u64 length + configuration text
 *   ("dim=", "experts=", "topk=" lines as config_text writes them, plus
 *   "moe_hidden=" for up/down experts: that shape has no reference key, so
 *   a new architecture key names it), u64 record count, the records, the
 *   trailer.
 * Parameter order of one layer (moe_layer_param_sizes): [LayerNorm gamma, beta,]
 * router [E][D], then per expert e: W_e [D][D] (hidden == 0, the reference's
 * order), or W_up[e] [h][D] followed by W_down[e] [D][h] (hidden > 0).
 * Errors throw std::runtime_error, as the reference's checkpoint code does.
 */
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <fstream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "tmt_moe.h"

namespace tmt_ckpt {

constexpr uint64_t kHashInit = UINT64_C(14695981039346656037);  // FNV-1a 64 offset basis
constexpr uint64_t kHashPrime = UINT64_C(1099511628211);
constexpr uint64_t kMagicV3 = UINT64_C(0x33544b5043544d54);      // "TMTCPKT3"

// 64-bit FNV-1a over `size` bytes, continuing from h.
inline uint64_t hash_bytes(uint64_t h, const void* data, size_t size) {
    const auto* b = static_cast<const unsigned char*>(data);
    for (size_t i = 0; i < size; ++i) h = (h ^ b[i]) * kHashPrime;
    return h;
}

// A hashed file stream; every byte written or read goes through bytes().
class Checkpoint {
public:
    Checkpoint(const std::string& path, bool write) : writing_(write) {
        file_ = std::fopen(path.c_str(), write ? "wb" : "rb");
        if (!file_) throw std::runtime_error("cannot open checkpoint: " + path);
    }
    ~Checkpoint() {
        if (file_) std::fclose(file_);
    }
    Checkpoint(const Checkpoint&) = delete;
    Checkpoint& operator=(const Checkpoint&) = delete;
    bool writing() const { return writing_; }
    void bytes(void* p, size_t n) {
        const size_t got = writing_ ? std::fwrite(p, 1, n, file_) : std::fread(p, 1, n, file_);
        if (got != n) throw std::runtime_error("checkpoint I/O failed or truncated");
        hash_ = hash_bytes(hash_, p, n);
    }
    template <class T>
    void scalar(T& v) {
        bytes(&v, sizeof(v));
    }
    // Device memory through bounded (1 MiB) host staging.
    void device(void* dev, size_t n) {
        std::vector<unsigned char> buf(n < (size_t(1) << 20) ? n : (size_t(1) << 20));
        for (size_t off = 0; off < n; off += buf.size()) {
            const size_t k = n - off < buf.size() ? n - off : buf.size();
            auto* g = static_cast<unsigned char*>(dev) + off;
            if (writing_) check(hipMemcpy(buf.data(), g, k, hipMemcpyDeviceToHost));
            bytes(buf.data(), k);
            if (!writing_) check(hipMemcpy(g, buf.data(), k, hipMemcpyHostToDevice));
        }
    }
    // Writer: append the hash. Reader: the trailer must equal the running
    // hash and be the last 8 bytes of the file.
    void finish() {
        uint64_t h = hash_;
        if (writing_) {
            if (std::fwrite(&h, sizeof(h), 1, file_) != 1 || std::fflush(file_))
                throw std::runtime_error("checkpoint flush failed");
        } else {
            uint64_t expected = 0;
            if (std::fread(&expected, sizeof(expected), 1, file_) != 1 || expected != h ||
                std::fgetc(file_) != EOF)
                throw std::runtime_error("checkpoint checksum/trailer mismatch");
        }
    }

private:
    static void check(hipError_t e) {
        if (e != hipSuccess) throw std::runtime_error(std::string("checkpoint copy: ") + hipGetErrorString(e));
    }
    std::FILE* file_ = nullptr;
    bool writing_;
    uint64_t hash_ = kHashInit;
};

// Whole-file integrity check before anything is loaded (checkpoint.h:59-73).
inline void verify_checkpoint(const std::string& path) {
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    if (!in) throw std::runtime_error("cannot read checkpoint");
    const auto size = in.tellg();
    if (size < std::streamoff(16)) throw std::runtime_error("checkpoint truncated");
    in.seekg(0);
    uint64_t remaining = (uint64_t)size - 8, h = kHashInit, expected = 0;
    std::vector<char> buf(65536);
    while (remaining) {
        const size_t n = remaining < buf.size() ? (size_t)remaining : buf.size();
        if (!in.read(buf.data(), (std::streamsize)n)) throw std::runtime_error("checkpoint read failed");
        h = hash_bytes(h, buf.data(), n);
        remaining -= n;
    }
    if (!in.read(reinterpret_cast<char*>(&expected), 8) || h != expected)
        throw std::runtime_error("checkpoint checksum mismatch");
}

// One parameter's device state, as the reference's Par (train.cu:35-41).
struct Param {
    float* master = nullptr;
    float* m = nullptr;
    float* v = nullptr;
    uint16_t* work = nullptr;  // bf16 copy for the kernels, or nullptr
    int64_t n = 0;
};

// The block's parameter shapes in registration order.
struct LayerShape {
    int dim = 0, experts = 0, topk = 0, hidden = 0;
    bool layernorm = false;  // gamma and beta precede the router (model.cu:222-231)
};
inline std::vector<int64_t> moe_layer_param_sizes(const LayerShape& s) {
    std::vector<int64_t> n;
    const int64_t D = s.dim;
    if (s.layernorm) {
        n.push_back(D);
        n.push_back(D);
    }
    n.push_back((int64_t)s.experts * D);
    for (int e = 0; e < s.experts; ++e) {
        if (s.hidden == 0) {
            n.push_back(D * D);
        } else {
            n.push_back((int64_t)s.hidden * D);
            n.push_back(D * (int64_t)s.hidden);
        }
    }
    return n;
}

// The configuration text of a block file ("key=value" lines).
inline std::string layer_config_text(const LayerShape& s) {
    std::ostringstream o;
    o << "dim=" << s.dim << "\n" << "experts=" << s.experts << "\n" << "topk=" << s.topk << "\n";
    if (s.hidden > 0) o << "moe_hidden=" << s.hidden << "\n";
    if (s.layernorm) o << "moe_layernorm=1\n";
    return o.str();
}

// The record loop of checkpoint_payload (checkpoint.h:143-150) over `ps`;
// on load the bf16 work copies are regenerated from the masters.
inline void param_records(Checkpoint& io, std::vector<Param>& ps, hipStream_t stream = nullptr) {
    uint64_t count = ps.size();
    io.scalar(count);
    if (count != ps.size()) throw std::runtime_error("checkpoint parameter count mismatch");
    for (auto& p : ps) {
        uint64_t n = (uint64_t)p.n;
        io.scalar(n);
        if (n != (uint64_t)p.n) throw std::runtime_error("checkpoint parameter shape mismatch");
        io.device(p.master, n * 4);
        io.device(p.m, n * 4);
        io.device(p.v, n * 4);
        if (!io.writing() && p.work) {
            if (tmt_moe_f32_to_bf16(stream, p.master, p.work, (int64_t)n) != TMT_MOE_OK)
                throw std::runtime_error(std::string("checkpoint work copy: ") + tmt_moe_last_error());
        }
    }
    if (!io.writing() && hipStreamSynchronize(stream) != hipSuccess)
        throw std::runtime_error("checkpoint work copy failed");
}

inline void layer_header(Checkpoint& io, const LayerShape& s) {
    uint64_t magic = kMagicV3;
    io.scalar(magic);
    if (magic != kMagicV3) throw std::runtime_error("unsupported checkpoint format");
    std::string text = layer_config_text(s);
    uint64_t len = text.size();
    io.scalar(len);
    if (len == 0 || len > 16384) throw std::runtime_error("invalid checkpoint configuration length");
    std::string got(len, '\0');
    if (io.writing()) got = text;
    io.bytes(&got[0], len);
    if (!io.writing() && got != text)
        throw std::runtime_error("checkpoint architecture differs: stored\n" + got + "expected\n" + text);
}

// Block file: header, records, trailer. The parameter list must follow
// moe_layer_param_sizes(s). Writes through a temporary name and renames, so
// a failed save leaves any previous file intact (checkpoint.h:167-173).
inline void save_layer(const std::string& path, const LayerShape& s, std::vector<Param>& ps) {
    const auto sizes = moe_layer_param_sizes(s);
    if (sizes.size() != ps.size()) throw std::runtime_error("parameter list does not match the layer shape");
    for (size_t i = 0; i < ps.size(); ++i)
        if (ps[i].n != sizes[i]) throw std::runtime_error("parameter size does not match the layer shape");
    const std::string tmp = path + ".tmp";
    try {
        {
            Checkpoint io(tmp, true);
            layer_header(io, s);
            param_records(io, ps);
            io.finish();
        }
        if (std::rename(tmp.c_str(), path.c_str())) throw std::runtime_error("checkpoint rename failed");
    } catch (...) {
        std::remove(tmp.c_str());
        throw;
    }
}

inline void load_layer(const std::string& path, const LayerShape& s, std::vector<Param>& ps,
                       hipStream_t stream = nullptr) {
    verify_checkpoint(path);  // before any parameter is touched
    const auto sizes = moe_layer_param_sizes(s);
    if (sizes.size() != ps.size()) throw std::runtime_error("parameter list does not match the layer shape");
    for (size_t i = 0; i < ps.size(); ++i)
        if (ps[i].n != sizes[i]) throw std::runtime_error("parameter size does not match the layer shape");
    Checkpoint io(path, false);
    layer_header(io, s);
    param_records(io, ps, stream);
    io.finish();
}

}  // namespace tmt_ckpt
