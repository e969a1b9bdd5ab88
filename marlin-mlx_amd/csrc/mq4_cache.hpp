// mq4_cache.hpp -- on-disk cache of MLX-affine Q4 weights (safetensors), for
// C++ callers of libmq4.
//
// The reference quantizes every MLP and lm_head weight when it loads the
// model (quantize_weight, src/model/weights.cpp:45-56; lm_head,
// src/model/weights.cpp:180-194).  save_q4_cache writes the quantized tensors
// once and load_q4_cache brings them back to the device, skipping the
// quantize step.  One safetensors file holds three tensors per matrix in
// MLX's naming convention -- "<name>.weight" U32 [N, K/8], "<name>.scales"
// and "<name>.biases" BF16 [N, K/64] -- and the group size and bit width in
// its metadata ("quantization.group_size", "quantization.bits").
//
// File layout (the public safetensors format): 8-byte little-endian header
// length, a JSON header {name: {"dtype", "shape", "data_offsets"}, ...,
// "__metadata__": {string: string}} padded with spaces to a multiple of 8,
// then the raw little-endian tensor bytes.  The reader accepts any file of
// that form (it parses the JSON subset the format uses: objects, strings,
// integer arrays); only local paths are used.
#pragma once

#include <cctype>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "mq4.hpp"

namespace mq4 {

// One tensor of a safetensors file, in host memory.
struct HostTensor {
    std::string dtype;              // "U32", "BF16", ...
    std::vector<int64_t> shape;
    std::vector<uint8_t> data;      // raw little-endian bytes
};

namespace cache_detail {

inline int64_t dtype_size(const std::string& dt) {
    if (dt == "U32" || dt == "I32" || dt == "F32") return 4;
    if (dt == "BF16" || dt == "F16" || dt == "U16" || dt == "I16") return 2;
    if (dt == "U8" || dt == "I8" || dt == "BOOL") return 1;
    if (dt == "F64" || dt == "I64" || dt == "U64") return 8;
    return 0;
}

// Minimal JSON reader for the safetensors header.
struct Json {
    enum Kind { NUL, NUM, STR, ARR, OBJ } kind = NUL;
    int64_t num = 0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json* get(const std::string& k) const {
        for (auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

class Parser {
public:
    explicit Parser(const std::string& s) : s_(s) {}
    bool parse(Json& out) {
        if (!value(out)) return false;
        ws();
        return i_ == s_.size();
    }

private:
    // A safetensors header nests three levels deep; the limit keeps a crafted
    // header from exhausting the stack through the recursion below.
    static constexpr int kMaxDepth = 32;
    const std::string& s_;
    size_t i_ = 0;
    int depth_ = 0;
    struct Nest {
        int& d;
        explicit Nest(int& d_) : d(++d_) {}
        ~Nest() { --d; }
    };
    void ws() {
        while (i_ < s_.size() && std::isspace((unsigned char)s_[i_])) ++i_;
    }
    bool string(std::string& out) {
        if (i_ >= s_.size() || s_[i_] != '"') return false;
        ++i_;
        while (i_ < s_.size() && s_[i_] != '"') {
            char c = s_[i_++];
            if (c == '\\') {
                if (i_ >= s_.size()) return false;
                char e = s_[i_++];
                switch (e) {
                    case 'n': c = '\n'; break;
                    case 't': c = '\t'; break;
                    case 'r': c = '\r'; break;
                    case 'b': c = '\b'; break;
                    case 'f': c = '\f'; break;
                    case 'u': {                         // keep ASCII, map others to '?'
                        if (i_ + 4 > s_.size()) return false;
                        const unsigned v = (unsigned)std::strtoul(s_.substr(i_, 4).c_str(), nullptr, 16);
                        i_ += 4;
                        c = v < 128 ? (char)v : '?';
                        break;
                    }
                    default: c = e;
                }
            }
            out.push_back(c);
        }
        if (i_ >= s_.size()) return false;
        ++i_;
        return true;
    }
    bool value(Json& v) {
        const Nest nest(depth_);
        if (depth_ > kMaxDepth) return false;
        ws();
        if (i_ >= s_.size()) return false;
        const char c = s_[i_];
        if (c == '{') {
            v.kind = Json::OBJ;
            ++i_;
            ws();
            if (i_ < s_.size() && s_[i_] == '}') { ++i_; return true; }
            for (;;) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (i_ >= s_.size() || s_[i_] != ':') return false;
                ++i_;
                Json e;
                if (!value(e)) return false;
                v.obj.emplace_back(std::move(k), std::move(e));
                ws();
                if (i_ < s_.size() && s_[i_] == ',') { ++i_; continue; }
                if (i_ < s_.size() && s_[i_] == '}') { ++i_; return true; }
                return false;
            }
        }
        if (c == '[') {
            v.kind = Json::ARR;
            ++i_;
            ws();
            if (i_ < s_.size() && s_[i_] == ']') { ++i_; return true; }
            for (;;) {
                Json e;
                if (!value(e)) return false;
                v.arr.push_back(std::move(e));
                ws();
                if (i_ < s_.size() && s_[i_] == ',') { ++i_; continue; }
                if (i_ < s_.size() && s_[i_] == ']') { ++i_; return true; }
                return false;
            }
        }
        if (c == '"') {
            v.kind = Json::STR;
            return string(v.str);
        }
        if (c == '-' || std::isdigit((unsigned char)c)) {
            v.kind = Json::NUM;
            size_t j = i_ + 1;
            while (j < s_.size() && std::isdigit((unsigned char)s_[j])) ++j;
            v.num = std::strtoll(s_.substr(i_, j - i_).c_str(), nullptr, 10);
            i_ = j;
            return true;
        }
        return false;
    }
};

inline std::string quote(const std::string& s) {
    std::string o = "\"";
    for (char c : s) {
        if (c == '"' || c == '\\') o.push_back('\\');
        o.push_back(c);
    }
    return o + "\"";
}

}  // namespace cache_detail

// Write named host tensors (in the given order) and string metadata.
inline Result<int> write_safetensors(const std::string& path,
                                     const std::vector<std::pair<std::string, HostTensor>>& tensors,
                                     const std::map<std::string, std::string>& metadata) {
    using namespace cache_detail;
    std::string h = "{";
    bool first = true;
    if (!metadata.empty()) {
        h += "\"__metadata__\":{";
        bool f2 = true;
        for (auto& kv : metadata) {
            h += (f2 ? "" : ",") + quote(kv.first) + ":" + quote(kv.second);
            f2 = false;
        }
        h += "}";
        first = false;
    }
    uint64_t off = 0;
    for (auto& [name, t] : tensors) {
        int64_t n = 1;
        for (int64_t d : t.shape) n *= d;
        if (dtype_size(t.dtype) == 0 || (uint64_t)(n * dtype_size(t.dtype)) != t.data.size())
            return Error{MQ4_ERR_INVALID_ARG, "write_safetensors: " + name + ": size does not match dtype and shape"};
        h += (first ? "" : ",") + quote(name) + ":{\"dtype\":" + quote(t.dtype) + ",\"shape\":[";
        for (size_t i = 0; i < t.shape.size(); ++i) h += (i ? "," : "") + std::to_string(t.shape[i]);
        h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + t.data.size()) + "]}";
        off += t.data.size();
        first = false;
    }
    h += "}";
    while (h.size() % 8) h.push_back(' ');
    const std::string tmp = path + ".tmp";
    FILE* f = std::fopen(tmp.c_str(), "wb");
    if (!f) return Error{MQ4_ERR_INVALID_ARG, "write_safetensors: cannot open " + tmp};
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)((uint64_t)h.size() >> (8 * i));
    bool ok = std::fwrite(len, 1, 8, f) == 8 && std::fwrite(h.data(), 1, h.size(), f) == h.size();
    for (auto& kv : tensors)
        ok = ok && std::fwrite(kv.second.data.data(), 1, kv.second.data.size(), f) == kv.second.data.size();
    ok = (std::fclose(f) == 0) && ok;
    if (!ok || std::rename(tmp.c_str(), path.c_str()) != 0)
        return Error{MQ4_ERR_INVALID_ARG, "write_safetensors: write to " + path + " failed"};
    return 0;
}

// Read every tensor of a safetensors file into host memory.
inline Result<std::map<std::string, HostTensor>> read_safetensors(const std::string& path,
                                                                   std::map<std::string, std::string>* metadata = nullptr) {
    using namespace cache_detail;
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return Error{MQ4_ERR_INVALID_ARG, "read_safetensors: cannot open " + path};
    uint8_t len[8];
    if (std::fread(len, 1, 8, f) != 8) { std::fclose(f); return Error{MQ4_ERR_INVALID_ARG, path + ": truncated"}; }
    uint64_t n = 0;
    for (int i = 0; i < 8; ++i) n |= (uint64_t)len[i] << (8 * i);
    std::fseek(f, 0, SEEK_END);
    const long fsize = std::ftell(f);
    if (fsize < 0 || n > (uint64_t)fsize - 8) { std::fclose(f); return Error{MQ4_ERR_INVALID_ARG, path + ": bad header length"}; }
    std::string hs(n, '\0');
    std::fseek(f, 8, SEEK_SET);
    if (std::fread(&hs[0], 1, n, f) != n) { std::fclose(f); return Error{MQ4_ERR_INVALID_ARG, path + ": truncated header"}; }
    const uint64_t data_size = (uint64_t)fsize - 8 - n;
    std::vector<uint8_t> data(data_size);
    if (data_size && std::fread(data.data(), 1, data_size, f) != data_size) {
        std::fclose(f);
        return Error{MQ4_ERR_INVALID_ARG, path + ": truncated data"};
    }
    std::fclose(f);
    Json root;
    if (!Parser(hs).parse(root) || root.kind != Json::OBJ) return Error{MQ4_ERR_INVALID_ARG, path + ": bad JSON header"};
    std::map<std::string, HostTensor> out;
    for (auto& [name, e] : root.obj) {
        if (name == "__metadata__") {
            if (metadata)
                for (auto& kv : e.obj)
                    if (kv.second.kind == Json::STR) (*metadata)[kv.first] = kv.second.str;
            continue;
        }
        const Json* dt = e.get("dtype");
        const Json* sh = e.get("shape");
        const Json* of = e.get("data_offsets");
        if (!dt || !sh || !of || dt->kind != Json::STR || sh->kind != Json::ARR || of->kind != Json::ARR ||
            of->arr.size() != 2)
            return Error{MQ4_ERR_INVALID_ARG, path + ": malformed entry " + name};
        HostTensor t;
        t.dtype = dt->str;
        // element and byte counts without overflow: each dimension is capped
        // and every product is checked, so no wrapped count can match the
        // data offsets while the dimensions disagree with the bytes
        constexpr int64_t kMaxDim = int64_t(1) << 40;
        int64_t cnt = 1, nbytes = 0;
        for (auto& d : sh->arr) {
            if (d.kind != Json::NUM || d.num < 0 || d.num > kMaxDim || __builtin_mul_overflow(cnt, d.num, &cnt))
                return Error{MQ4_ERR_INVALID_ARG, path + ": bad shape of " + name};
            t.shape.push_back(d.num);
        }
        const int64_t b = of->arr[0].num, en = of->arr[1].num;
        if (of->arr[0].kind != Json::NUM || of->arr[1].kind != Json::NUM || b < 0 || en < b ||
            (uint64_t)en > data_size || dtype_size(t.dtype) == 0 ||
            __builtin_mul_overflow(cnt, dtype_size(t.dtype), &nbytes) || en - b != nbytes)
            return Error{MQ4_ERR_INVALID_ARG, path + ": data offsets of " + name + " do not match its shape"};
        t.data.assign(data.begin() + b, data.begin() + en);
        out.emplace(name, std::move(t));
    }
    return out;
}

// A quantized matrix copied to host memory, as the cache stores it.
inline Result<int> q4_to_host(const QuantizedTensor& q, HostTensor& w, HostTensor& s, HostTensor& b) {
    if (!q.quantized) return Error{MQ4_ERR_INVALID_ARG, "q4_to_host: not a quantized tensor"};
    const int64_t N = q.out_features, K = q.in_features, G = K / q.group_size;
    w = {"U32", {N, K * q.bits / 32}, std::vector<uint8_t>((size_t)(N * K * q.bits / 8))};
    s = {"BF16", {N, G}, std::vector<uint8_t>((size_t)(N * G * 2))};
    b = {"BF16", {N, G}, std::vector<uint8_t>((size_t)(N * G * 2))};
    if (hipMemcpy(w.data.data(), q.weight.get(), w.data.size(), hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(s.data.data(), q.scales.get(), s.data.size(), hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(b.data.data(), q.biases.get(), b.data.size(), hipMemcpyDeviceToHost) != hipSuccess)
        return Error{MQ4_ERR_HIP, "q4_to_host: hipMemcpy failed"};
    return 0;
}

// Save named quantized matrices (device) to one safetensors file.
inline Result<int> save_q4_cache(const std::string& path,
                                 const std::vector<std::pair<std::string, const QuantizedTensor*>>& mats) {
    std::vector<std::pair<std::string, HostTensor>> ts;
    int gs = 64, bits = 4;
    for (auto& [name, q] : mats) {
        HostTensor w, s, b;
        auto r = q4_to_host(*q, w, s, b);
        if (!r) return r.error();
        gs = q->group_size;
        bits = q->bits;
        ts.emplace_back(name + ".weight", std::move(w));
        ts.emplace_back(name + ".scales", std::move(s));
        ts.emplace_back(name + ".biases", std::move(b));
    }
    return write_safetensors(path, ts, {{"format", "mlx"}, {"quantization.group_size", std::to_string(gs)},
                                        {"quantization.bits", std::to_string(bits)}});
}

// The group size and bit width a cache file records (64 and 4 when absent).
// MLX also writes group 32 / 128 and 2, 3, 6 or 8 bits; the library's kernels
// read only the group-64, 4-bit layout, so any other format is refused here,
// before its buffers could reach an entry point that assumes that layout.
inline Result<int> q4_cache_format(const std::map<std::string, std::string>& meta, const std::string& path) {
    auto num = [&](const char* key, int dflt) {
        auto it = meta.find(key);
        return it == meta.end() ? dflt : std::atoi(it->second.c_str());
    };
    const int gs = num("quantization.group_size", 64), bits = num("quantization.bits", 4);
    if (gs != 64 || bits != 4)
        return Error{MQ4_ERR_UNSUPPORTED, path + ": holds group_size=" + std::to_string(gs) + ", bits=" +
                                              std::to_string(bits) + "; only group_size=64, bits=4 is implemented"};
    return 0;
}

// Load every "<name>.weight/.scales/.biases" triple of a cache file to the
// device (shapes and dtypes checked against the group-64, 4-bit layout).
inline Result<std::map<std::string, QuantizedTensor>> load_q4_cache(const std::string& path) {
    std::map<std::string, std::string> meta;
    auto rr = read_safetensors(path, &meta);
    if (!rr) return rr.error();
    auto& t = rr.value();
    if (auto fr = q4_cache_format(meta, path); !fr) return fr.error();
    const int gs = 64, bits = 4;
    std::map<std::string, QuantizedTensor> out;
    const std::string suf = ".weight";
    for (auto& [key, w] : t) {
        if (key.size() <= suf.size() || key.compare(key.size() - suf.size(), suf.size(), suf) != 0) continue;
        const std::string name = key.substr(0, key.size() - suf.size());
        auto si = t.find(name + ".scales"), bi = t.find(name + ".biases");
        if (si == t.end() || bi == t.end()) continue;
        const HostTensor &s = si->second, &b = bi->second;
        if (w.dtype != "U32" || s.dtype != "BF16" || b.dtype != "BF16" || w.shape.size() != 2 || s.shape.size() != 2 ||
            s.shape != b.shape || s.shape[0] != w.shape[0])
            return Error{MQ4_ERR_INVALID_ARG, path + ": " + name + ": unexpected dtypes or shapes"};
        const int64_t N = w.shape[0], K = w.shape[1] * 32 / bits;
        if (K % gs != 0 || s.shape[1] != K / gs)
            return Error{MQ4_ERR_INVALID_ARG, path + ": " + name + ": scales do not match K and the group size"};
        QuantizedTensor q;
        q.out_features = N;
        q.in_features = K;
        q.group_size = gs;
        q.bits = bits;
        q.weight = DeviceBuffer(w.data.size());
        q.scales = DeviceBuffer(s.data.size());
        q.biases = DeviceBuffer(b.data.size());
        if (!q.weight.get() || !q.scales.get() || !q.biases.get() ||
            hipMemcpy(q.weight.get(), w.data.data(), w.data.size(), hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(q.scales.get(), s.data.data(), s.data.size(), hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(q.biases.get(), b.data.data(), b.data.size(), hipMemcpyHostToDevice) != hipSuccess)
            return Error{MQ4_ERR_HIP, "load_q4_cache: device upload of " + name + " failed"};
        q.quantized = true;
        out.emplace(name, std::move(q));
    }
    return out;
}

}  // namespace mq4
