// test_ckpt.cpp -- the block's parameters in the V3 checkpoint layout
// (include/tmt_moe_ckpt.hpp), in the style of the reference's checkpoint
// checks (tmt-cuda/src/architecture_test.cu:125-141: exact resume and a
// corrupted file rejected).
//
// Usage: test_ckpt host   format checks on host memory only (no GPU)
//        test_ckpt        all checks, including device round trips
#include "tmt_moe_ckpt.hpp"

#include <cmath>
#include <cstring>
#include <random>
#include <string>
#include <unistd.h>
#include <vector>

static void require(bool ok, const char* what) {
    if (!ok) {
        std::printf("FAIL %s\n", what);
        std::exit(1);
    }
}

static std::string tmp_path(const char* tag) {
    return "/tmp/tmt-moe-ckpt-" + std::to_string(getpid()) + "-" + tag;
}

static bool throws(void (*f)(const std::string&), const std::string& arg) {
    try {
        f(arg);
    } catch (const std::exception&) {
        return true;
    }
    return false;
}

static void write_raw(const std::string& path, const std::vector<unsigned char>& bytes) {
    FILE* f = std::fopen(path.c_str(), "wb");
    require(f && std::fwrite(bytes.data(), 1, bytes.size(), f) == bytes.size(), "raw write");
    std::fclose(f);
}

static std::vector<unsigned char> read_raw(const std::string& path) {
    FILE* f = std::fopen(path.c_str(), "rb");
    require(f != nullptr, "raw open");
    std::vector<unsigned char> b;
    int c;
    while ((c = std::fgetc(f)) != EOF) b.push_back((unsigned char)c);
    std::fclose(f);
    return b;
}

// FNV-1a 64 known answers (the published test vectors of the algorithm),
// a hand-built file checked byte by byte, and damaged files refused.
static void test_host_format() {
    using tmt_ckpt::fnv1a64;
    require(fnv1a64("", 0) == UINT64_C(0xcbf29ce484222325), "FNV-1a of the empty string");
    require(fnv1a64("a", 1) == UINT64_C(0xaf63dc4c8601ec8c), "FNV-1a of \"a\"");
    require(fnv1a64("foobar", 6) == UINT64_C(0x85944171f73967e8), "FNV-1a of \"foobar\"");
    require(fnv1a64("bar", 3, fnv1a64("foo", 3)) == fnv1a64("foobar", 6), "FNV-1a streams");
    const std::string path = tmp_path("host");
    {
        tmt_ckpt::Writer w(path);
        w.put_u64(tmt_ckpt::kMagic);
        const float vals[3] = {1.f, -2.f, 3.5f};
        w.put(vals, sizeof vals);
        w.commit();
    }
    tmt_ckpt::check_file(path);
    std::vector<unsigned char> b = read_raw(path);
    require(b.size() == 8 + 12 + 8, "file = magic + payload + 8-byte trailer");
    require(std::memcmp(b.data(), "TMTCPKT3", 8) == 0, "magic bytes spell TMTCPKT3");
    uint64_t trailer;
    std::memcpy(&trailer, b.data() + 20, 8);
    require(trailer == fnv1a64(b.data(), 20), "trailer is the FNV-1a hash of all preceding bytes");
    {
        std::vector<unsigned char> bad = b;
        bad[9] ^= 1;
        write_raw(path, bad);
        require(throws(tmt_ckpt::check_file, path), "a flipped bit is rejected");
        bad = b;
        bad.push_back(0);
        write_raw(path, bad);
        require(throws(tmt_ckpt::check_file, path), "a byte after the trailer is rejected");
        write_raw(path, std::vector<unsigned char>(b.begin(), b.begin() + 5));
        require(throws(tmt_ckpt::check_file, path), "a truncated file is rejected");
    }
    {
        // a writer that never commits leaves no file behind
        const std::string p2 = tmp_path("uncommitted");
        {
            tmt_ckpt::Writer w(p2);
            w.put_u64(1);
        }
        require(std::fopen(p2.c_str(), "rb") == nullptr, "an uncommitted write leaves no file");
    }
    std::remove(path.c_str());
    tmt_ckpt::LayerShape s;
    s.dim = 64; s.experts = 4; s.topk = 2;
    auto sz = tmt_ckpt::moe_layer_param_sizes(s);
    require(sz.size() == 5 && sz[0] == 256 && sz[1] == 64 * 64, "reference layer order: router, then W_e");
    require(tmt_ckpt::layer_config_text(s) == "dim=64\nexperts=4\ntopk=2\n", "configuration text keys");
    s.hidden = 128; s.layernorm = true;
    sz = tmt_ckpt::moe_layer_param_sizes(s);
    require(sz.size() == 2 + 1 + 8 && sz[0] == 64 && sz[2] == 256 && sz[3] == 128 * 64 && sz[4] == 64 * 128,
            "gamma, beta, router, then W_up[e], W_down[e] per expert");
    std::puts("PASS checkpoint format: FNV-1a vectors, trailer, corruption, extra bytes and truncation rejected");
}

struct DevParams {
    std::vector<tmt_ckpt::Param> ps;
    std::vector<void*> bufs;
    ~DevParams() {
        for (void* b : bufs) (void)hipFree(b);
    }
    void add(int64_t n, std::mt19937& g) {
        tmt_ckpt::Param p;
        p.n = n;
        std::normal_distribution<float> nd(0.f, 1.f);
        std::vector<float> h(n);
        float** dst[3] = {&p.master, &p.m, &p.v};
        for (float** d : dst) {
            for (auto& x : h) x = nd(g);
            void* b = nullptr;
            require(hipMalloc(&b, n * 4) == hipSuccess, "hipMalloc");
            require(hipMemcpy(b, h.data(), n * 4, hipMemcpyHostToDevice) == hipSuccess, "upload");
            bufs.push_back(b);
            *d = (float*)b;
        }
        void* w = nullptr;
        require(hipMalloc(&w, n * 2) == hipSuccess, "hipMalloc");
        require(hipMemset(w, 0xff, n * 2) == hipSuccess, "hipMemset");
        bufs.push_back(w);
        p.work = (uint16_t*)w;
        ps.push_back(p);
    }
};

static std::vector<float> dl(const float* p, int64_t n) {
    std::vector<float> v(n);
    require(hipMemcpy(v.data(), p, n * 4, hipMemcpyDeviceToHost) == hipSuccess, "download");
    return v;
}

static void round_trip(tmt_ckpt::LayerShape s, const char* tag) {
    std::mt19937 g(3);
    DevParams a, b;
    for (int64_t n : tmt_ckpt::moe_layer_param_sizes(s)) {
        a.add(n, g);
        b.add(n, g);
    }
    const std::string path = tmp_path(tag);
    tmt_ckpt::save_layer(path, s, a.ps);
    // size: magic + length + text + count + records (n + 3 fp32 arrays each) + trailer
    int64_t expect = 8 + 8 + (int64_t)tmt_ckpt::layer_config_text(s).size() + 8 + 8;
    for (auto& p : a.ps) expect += 8 + 12 * p.n;
    FILE* f = std::fopen(path.c_str(), "rb");
    std::fseek(f, 0, SEEK_END);
    require(std::ftell(f) == expect, "file size follows the V3 record layout");
    std::fclose(f);
    tmt_ckpt::load_layer(path, s, b.ps);
    for (size_t i = 0; i < a.ps.size(); ++i) {
        const int64_t n = a.ps[i].n;
        require(dl(a.ps[i].master, n) == dl(b.ps[i].master, n), "master weights round-trip exactly");
        require(dl(a.ps[i].m, n) == dl(b.ps[i].m, n) && dl(a.ps[i].v, n) == dl(b.ps[i].v, n),
                "Adam moments round-trip exactly");
        std::vector<uint16_t> w(n);
        require(hipMemcpy(w.data(), b.ps[i].work, n * 2, hipMemcpyDeviceToHost) == hipSuccess, "download");
        auto m = dl(b.ps[i].master, n);
        for (int64_t k = 0; k < n; ++k) {
            uint32_t u;
            std::memcpy(&u, &m[k], 4);
            const uint16_t want = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
            require(w[k] == want, "bf16 work copy regenerated from the master (round to nearest even)");
        }
    }
    // a different architecture is refused before anything changes
    tmt_ckpt::LayerShape other = s;
    other.topk = s.topk + 1;
    bool refused = false;
    try {
        tmt_ckpt::load_layer(path, other, b.ps);
    } catch (const std::exception&) {
        refused = true;
    }
    require(refused, "a checkpoint of another architecture is refused");
    // a file cut inside the records but given a valid trailer again is
    // refused by the parser (the trailer alone does not catch it)
    {
        std::vector<unsigned char> bytes = read_raw(path);
        bytes.resize(bytes.size() - 8 - 40);
        const uint64_t h = tmt_ckpt::fnv1a64(bytes.data(), bytes.size());
        const unsigned char* hp = reinterpret_cast<const unsigned char*>(&h);
        bytes.insert(bytes.end(), hp, hp + 8);
        const std::string cut = tmp_path("cut");
        write_raw(cut, bytes);
        tmt_ckpt::check_file(cut);  // the trailer matches
        bool cut_refused = false;
        try {
            tmt_ckpt::load_layer(cut, s, b.ps);
        } catch (const std::exception&) {
            cut_refused = true;
        }
        require(cut_refused, "a file cut inside the records is refused");
        std::remove(cut.c_str());
    }
    // corruption: flip one byte in the middle; the load is refused and the
    // parameters keep their values
    f = std::fopen(path.c_str(), "r+b");
    std::fseek(f, expect / 2, SEEK_SET);
    const int c = std::fgetc(f);
    std::fseek(f, expect / 2, SEEK_SET);
    std::fputc(c ^ 0x10, f);
    std::fclose(f);
    std::mt19937 g2(9);
    DevParams fresh;
    for (int64_t n : tmt_ckpt::moe_layer_param_sizes(s)) fresh.add(n, g2);
    const auto before = dl(fresh.ps[0].master, fresh.ps[0].n);
    refused = false;
    try {
        tmt_ckpt::load_layer(path, s, fresh.ps);
    } catch (const std::exception&) {
        refused = true;
    }
    require(refused, "corrupted checkpoint accepted");
    require(dl(fresh.ps[0].master, fresh.ps[0].n) == before, "a refused load changed the parameters");
    std::remove(path.c_str());
    std::printf("PASS checkpoint round trip (%s): records exact, work copies regenerated, corruption and other architectures refused\n",
                tag);
}

int main(int argc, char** argv) {
    test_host_format();
    if (argc > 1 && std::string(argv[1]) == "host") {
        std::puts("HOST PASS");
        return 0;
    }
    tmt_ckpt::LayerShape ref;
    ref.dim = 64; ref.experts = 4; ref.topk = 2;
    round_trip(ref, "reference-experts");
    tmt_ckpt::LayerShape up;
    up.dim = 128; up.experts = 8; up.topk = 2; up.hidden = 256; up.layernorm = true;
    round_trip(up, "up-down-experts-with-layernorm");
    std::puts("ALL PASS");
    return 0;
}
