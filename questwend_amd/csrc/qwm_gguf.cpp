// qwm_gguf.cpp -- the tensor index of a GGUF model file, enough to find the
// expert slabs in it: Model::tensor_file_offset (core/model.cpp:454-458,
// 636-677) is the data section's offset plus the tensor's offset, where the
// data section starts at the end of the tensor infos rounded up to
// general.alignment (32 when absent; third_party/ggml/include/gguf.h:26-46).
// Layout read here (version 2 or 3, little endian):
//   "GGUF", u32 version, u64 n_tensors, u64 n_kv,
//   n_kv x (string key, u32 type, value), string = u64 length + bytes,
//   array value = u32 element type, u64 count, elements (no nested arrays),
//   n_tensors x (string name, u32 n_dims, n_dims x u64 ne, u32 ggml type,
//   u64 offset relative to the data section).
// The KV values are skipped except general.alignment.  Host code.
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "qwm_internal.h"

using namespace qwm;

namespace {

struct GgufTensor {
    int32_t type = 0, n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0;   // absolute
};

// ggml block sizes and bytes per block (ggml.c type_traits) of the types a
// model file's weights use; 0 bytes for the others.
void type_size(int32_t type, int64_t & blck, int64_t & bytes) {
    switch (type) {
        case 0: blck = 1; bytes = 4; return;      // F32
        case 1: blck = 1; bytes = 2; return;      // F16
        case 2: blck = 32; bytes = 18; return;    // Q4_0
        case 3: blck = 32; bytes = 20; return;    // Q4_1
        case 6: blck = 32; bytes = 22; return;    // Q5_0
        case 7: blck = 32; bytes = 24; return;    // Q5_1
        case 8: blck = 32; bytes = 34; return;    // Q8_0
        case 10: blck = 256; bytes = 84; return;  // Q2_K
        case 11: blck = 256; bytes = 110; return; // Q3_K
        case 12: blck = 256; bytes = 144; return; // Q4_K
        case 13: blck = 256; bytes = 176; return; // Q5_K
        case 14: blck = 256; bytes = 210; return; // Q6_K
        case 30: blck = 1; bytes = 2; return;     // BF16
        default: blck = 1; bytes = 0; return;
    }
}

class Reader {
public:
    explicit Reader(FILE * f) : f_(f) {
        std::fseek(f_, 0, SEEK_END);
        size_ = (uint64_t)std::ftell(f_);
        std::fseek(f_, 0, SEEK_SET);
    }
    bool raw(void * dst, size_t n) {
        if (pos_ + n > size_) return false;
        if (std::fread(dst, 1, n, f_) != n) return false;
        pos_ += n;
        return true;
    }
    template <class T> bool get(T & v) { return raw(&v, sizeof(T)); }
    bool skip(uint64_t n) {
        if (n > size_ - pos_) return false;
        pos_ += n;
        return std::fseek(f_, (long)pos_, SEEK_SET) == 0;
    }
    bool str(std::string & s) {
        uint64_t n = 0;
        if (!get(n) || n > size_ - pos_) return false;
        s.resize(n);
        return n == 0 || raw(&s[0], n);
    }
    uint64_t pos() const { return pos_; }

private:
    FILE * f_;
    uint64_t size_ = 0, pos_ = 0;
};

// bytes of one scalar KV value of GGUF type t (0: not a fixed-size scalar)
uint64_t scalar_bytes(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: return 0;
    }
}

bool skip_value(Reader & r, uint32_t t) {
    if (t == 8) {
        uint64_t n = 0;
        return r.get(n) && r.skip(n);
    }
    if (t == 9) {
        uint32_t et = 0;
        uint64_t n = 0;
        if (!r.get(et) || !r.get(n) || et == 9) return false;   // nested arrays are not GGUF
        if (et == 8) {
            for (uint64_t i = 0; i < n; ++i)
                if (!skip_value(r, 8)) return false;
            return true;
        }
        const uint64_t b = scalar_bytes(et);
        return b && n <= UINT64_MAX / b && r.skip(n * b);
    }
    const uint64_t b = scalar_bytes(t);
    return b && r.skip(b);
}

int read_index(const char * path, std::unordered_map<std::string, GgufTensor> & out) {
    FILE * f = std::fopen(path, "rb");
    if (!f) return fail(QWM_ERR_IO, std::string("gguf: ") + path + ": " + strerror(errno));
    Reader r(f);
    auto bad = [&](const std::string & why) {
        std::fclose(f);
        return fail(QWM_ERR_ARG, std::string("gguf: ") + path + ": " + why);
    };
    char magic[4];
    uint32_t version = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    if (!r.raw(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return bad("not a GGUF file");
    if (!r.get(version) || (version != 2 && version != 3)) return bad("unsupported version");
    if (!r.get(n_tensors) || !r.get(n_kv)) return bad("truncated header");
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key;
        uint32_t t = 0;
        if (!r.str(key) || !r.get(t)) return bad("truncated key/value section");
        if (key == "general.alignment") {
            uint32_t a = 0;
            if (t != 4 || !r.get(a) || a == 0 || (a & (a - 1))) return bad("general.alignment must be a power-of-two u32");
            alignment = a;
        } else if (!skip_value(r, t)) {
            return bad("malformed value of key " + key);
        }
    }
    std::vector<std::pair<std::string, GgufTensor>> infos;
    for (uint64_t i = 0; i < n_tensors; ++i) {
        std::string name;
        GgufTensor ti;
        uint32_t nd = 0;
        if (!r.str(name) || !r.get(nd) || nd < 1 || nd > 4) return bad("malformed tensor info");
        ti.n_dims = (int32_t)nd;
        for (uint32_t d = 0; d < nd; ++d) {
            uint64_t v = 0;
            if (!r.get(v) || v > (uint64_t)INT64_MAX) return bad("malformed tensor info");
            ti.ne[d] = (int64_t)v;
        }
        uint32_t type = 0;
        if (!r.get(type) || !r.get(ti.offset)) return bad("malformed tensor info");
        ti.type = (int32_t)type;
        infos.emplace_back(std::move(name), ti);
    }
    const uint64_t data = (r.pos() + alignment - 1) / alignment * alignment;
    std::fclose(f);
    for (auto & it : infos) {
        it.second.offset += data;
        out[it.first] = it.second;
    }
    return QWM_OK;
}

uint64_t tensor_bytes(const GgufTensor & t) {
    int64_t blck = 1, bytes = 0;
    type_size(t.type, blck, bytes);
    if (!bytes || t.ne[0] % blck) return 0;
    return (uint64_t)(t.ne[0] / blck * bytes) * (uint64_t)t.ne[1] * (uint64_t)t.ne[2] * (uint64_t)t.ne[3];
}

}  // namespace

extern "C" {

int qwm_gguf_find_tensor(const char * path, const char * name, qwm_gguf_tensor * out) {
    return guard("qwm_gguf_find_tensor", [&]() -> int {
        if (!path || !name || !out) return fail(QWM_ERR_ARG, "gguf_find_tensor: NULL argument");
        std::unordered_map<std::string, GgufTensor> idx;
        const int rc = read_index(path, idx);
        if (rc != QWM_OK) return rc;
        auto it = idx.find(name);
        if (it == idx.end()) return fail(QWM_ERR_ARG, std::string("gguf: no tensor ") + name + " in " + path);
        const GgufTensor & t = it->second;
        out->type = t.type;
        out->n_dims = t.n_dims;
        for (int d = 0; d < 4; ++d) out->ne[d] = t.ne[d];
        out->offset = t.offset;
        out->nbytes = tensor_bytes(t);
        return QWM_OK;
    });
}

int qwm_pool_attach_gguf(qwm_pool * pool, const char * path, int32_t first_block) {
    return guard("qwm_pool_attach_gguf", [&]() -> int {
        if (!pool || !path || first_block < 0) return fail(QWM_ERR_ARG, "pool_attach_gguf: bad argument");
        std::unordered_map<std::string, GgufTensor> idx;
        const int rc = read_index(path, idx);
        if (rc != QWM_OK) return rc;
        const int32_t n_layer = pool_n_layer(pool), n_expert = pool_n_expert(pool);
        static const char * const roles[3] = {"gate", "up", "down"};   // expert_cache.cpp:88-93
        for (int32_t l = 0; l < n_layer; ++l)
            for (int r = 0; r < 3; ++r) {
                const std::string name = "blk." + std::to_string(first_block + l) + ".ffn_" + roles[r] + "_exps.weight";
                auto it = idx.find(name);
                if (it == idx.end()) return fail(QWM_ERR_ARG, "gguf: no tensor " + name + " in " + path);
                const GgufTensor & t = it->second;
                const uint64_t nb = tensor_bytes(t);
                if (t.ne[2] != n_expert || t.ne[3] != 1 || nb != (uint64_t)n_expert * pool_slab_bytes(pool, r, l))
                    return fail(QWM_ERR_ARG, "gguf: " + name + " does not hold n_expert slabs of its pool's slab_bytes");
                const int arc = qwm_pool_attach_file(pool, r, l, path, t.offset);
                if (arc != QWM_OK) return arc;
            }
        return QWM_OK;
    });
}

}  // extern "C"
