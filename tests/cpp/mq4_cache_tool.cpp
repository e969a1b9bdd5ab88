// Host-side check of marlin-mlx_amd/csrc/mq4_cache.hpp (no GPU needed):
//   mq4_cache_tool write <path>   writes a fixed set of tensors with the C++ writer
//   mq4_cache_tool dump <path>    reads a file with the C++ reader and prints, per
//                                 tensor (sorted by name): name dtype shape fnv1a64(bytes)
//   mq4_cache_tool check <path>   reads a file and applies load_q4_cache's format
//                                 check (group 64, 4 bits); exit 0 if accepted
// tests/test_q4cache.py compares both directions with the Python module and
// with the safetensors library.
#include <cstdio>
#include <cstring>

#include "mq4_cache.hpp"

static uint64_t fnv1a(const std::vector<uint8_t>& d) {
    uint64_t h = 1469598103934665603ull;
    for (uint8_t c : d) {
        h ^= c;
        h *= 1099511628211ull;
    }
    return h;
}

int main(int argc, char** argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: %s write|dump|check <path>\n", argv[0]);
        return 2;
    }
    const std::string mode = argv[1], path = argv[2];
    if (mode == "write") {
        // layer.0.mlp.gate_proj: N=3, K=128 (words [3, 16], scales/biases [3, 2])
        std::vector<std::pair<std::string, mq4::HostTensor>> ts;
        mq4::HostTensor w{"U32", {3, 16}, std::vector<uint8_t>(3 * 16 * 4)};
        mq4::HostTensor s{"BF16", {3, 2}, std::vector<uint8_t>(3 * 2 * 2)};
        mq4::HostTensor b{"BF16", {3, 2}, std::vector<uint8_t>(3 * 2 * 2)};
        for (size_t i = 0; i < w.data.size(); ++i) w.data[i] = (uint8_t)(i * 37 + 11);
        for (size_t i = 0; i < s.data.size(); ++i) s.data[i] = (uint8_t)(i * 13 + 60);
        for (size_t i = 0; i < b.data.size(); ++i) b.data[i] = (uint8_t)(i * 7 + 190);
        ts.emplace_back("layer.0.mlp.gate_proj.weight", w);
        ts.emplace_back("layer.0.mlp.gate_proj.scales", s);
        ts.emplace_back("layer.0.mlp.gate_proj.biases", b);
        auto r = mq4::write_safetensors(path, ts, {{"format", "mlx"}, {"quantization.group_size", "64"},
                                                   {"quantization.bits", "4"}});
        if (!r) {
            std::fprintf(stderr, "%s\n", r.error().message.c_str());
            return 1;
        }
        return 0;
    }
    if (mode == "check") {
        std::map<std::string, std::string> meta;
        auto r = mq4::read_safetensors(path, &meta);
        if (!r) {
            std::fprintf(stderr, "%s\n", r.error().message.c_str());
            return 1;
        }
        auto f = mq4::q4_cache_format(meta, path);
        if (!f) {
            std::fprintf(stderr, "error %d: %s\n", f.error().code, f.error().message.c_str());
            return 3;
        }
        return 0;
    }
    if (mode == "dump") {
        std::map<std::string, std::string> meta;
        auto r = mq4::read_safetensors(path, &meta);
        if (!r) {
            std::fprintf(stderr, "%s\n", r.error().message.c_str());
            return 1;
        }
        for (auto& [k, v] : meta) std::printf("meta %s %s\n", k.c_str(), v.c_str());
        for (auto& [name, t] : r.value()) {
            std::printf("%s %s", name.c_str(), t.dtype.c_str());
            for (int64_t d : t.shape) std::printf(" %lld", (long long)d);
            std::printf(" %016llx\n", (unsigned long long)fnv1a(t.data));
        }
        return 0;
    }
    return 2;
}
