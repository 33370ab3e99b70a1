// safetensors.cpp -- model.safetensors reader behind ebh_load_safetensors.
//
// Replaces ModelWeights::load (src/weights.rs:15-45).  File layout: an
// 8-byte little-endian header length N, N bytes of JSON mapping each tensor
// name to {"dtype", "shape", "data_offsets": [begin, end]} (offsets relative
// to the end of the header), optional "__metadata__", then the raw data.
// The reference decodes every tensor as f32 LE whatever its dtype
// (src/weights.rs:25-29); here F32 is taken as-is and F16 / BF16 are widened
// exactly, any other dtype of a tensor the encoder needs is an error, and
// tensors the encoder does not use are skipped.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/edgebert_hip.h"
#include "internal.hpp"
#include "json.hpp"

namespace {

using ebh::json::JVal;
using ebh::json::Parser;


float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: renormalise
            exp = 127 - 15 + 1;
            while (!(man & 0x400u)) { man <<= 1; --exp; }
            bits = sign | (exp << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

float bf16_to_float(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

int fail(int code, const char* msg) { return ebh::set_error(code, "%s", msg); }

}  // namespace

extern "C" int ebh_load_safetensors(ebh_model* m, const char* path) {
    if (!m || !path) return fail(EBH_ERR_INVALID_ARG, "null argument");
    std::unique_ptr<FILE, int (*)(FILE*)> f(fopen(path, "rb"), fclose);
    if (!f) return fail(EBH_ERR_NOT_FOUND, (std::string("cannot open ") + path).c_str());
    uint8_t lenb[8];
    if (fread(lenb, 1, 8, f.get()) != 8) return fail(EBH_ERR_SHAPE, "safetensors: truncated header");
    uint64_t n = 0;
    for (int i = 7; i >= 0; --i) n = (n << 8) | lenb[i];
    if (n > (100u << 20)) return fail(EBH_ERR_SHAPE, "safetensors: header too large");
    std::string header(n, '\0');
    if (fread(&header[0], 1, n, f.get()) != n) return fail(EBH_ERR_SHAPE, "safetensors: truncated header");
    if (fseek(f.get(), 0, SEEK_END) != 0) return fail(EBH_ERR_SHAPE, "safetensors: seek failed");
    const long fsize = ftell(f.get());
    const uint64_t data_start = 8 + n;
    if (fsize < 0 || (uint64_t)fsize < data_start) return fail(EBH_ERR_SHAPE, "safetensors: truncated file");
    const uint64_t data_len = (uint64_t)fsize - data_start;

    Parser ps{header.data(), header.data() + header.size(), {}};
    JVal root;
    if (!ps.parse(root) || root.kind != JVal::OBJ)
        return fail(EBH_ERR_SHAPE, ("safetensors: bad header JSON: " + ps.err).c_str());

    ebh_config cfg;
    ebh_model_info(m, &cfg, nullptr);
    std::vector<float> buf;
    std::vector<uint8_t> raw;
    for (auto& kv : root.obj) {
        const std::string& name = kv.first;
        if (name == "__metadata__") continue;
        const JVal& t = kv.second;
        if (t.kind != JVal::OBJ || !t.obj.count("dtype") || !t.obj.count("shape") || !t.obj.count("data_offsets"))
            return fail(EBH_ERR_SHAPE, ("safetensors: malformed entry " + name).c_str());
        // The encoder's tensors and the cross-encoder head; pooler / position_ids are skipped.
        const bool wanted = name.rfind("embeddings.", 0) == 0 || name.rfind("encoder.layer.", 0) == 0 ||
                            name == "classifier.weight" || name == "classifier.bias";
        if (!wanted || name == "embeddings.position_ids") continue;
        const std::string& dt = t.obj.at("dtype").str;
        const JVal& shp = t.obj.at("shape");
        const JVal& offs = t.obj.at("data_offsets");
        if (shp.kind != JVal::ARR || offs.kind != JVal::ARR || offs.arr.size() != 2)
            return fail(EBH_ERR_SHAPE, ("safetensors: malformed entry " + name).c_str());
        std::vector<int64_t> shape;
        uint64_t count = 1;
        for (auto& d : shp.arr) {
            // Dimensions are non-negative integers; 2^40 bounds the element
            // count of any tensor this model could hold.
            if (d.kind != JVal::NUM || !(d.num >= 0.0) || d.num != (double)(int64_t)d.num ||
                d.num > (double)(1ull << 40))
                return fail(EBH_ERR_SHAPE, ("safetensors: bad shape for " + name).c_str());
            shape.push_back((int64_t)d.num);
            count *= (uint64_t)d.num;
            if (count > (1ull << 40))
                return fail(EBH_ERR_SHAPE, ("safetensors: bad shape for " + name).c_str());
        }
        for (auto& o : offs.arr)
            if (o.kind != JVal::NUM || !(o.num >= 0.0) || o.num > 9.0e15)
                return fail(EBH_ERR_SHAPE, ("safetensors: bad data_offsets for " + name).c_str());
        const uint64_t b0 = (uint64_t)offs.arr[0].num, b1 = (uint64_t)offs.arr[1].num;
        const int esz = dt == "F32" ? 4 : (dt == "F16" || dt == "BF16") ? 2 : 0;
        if (!esz)
            return fail(EBH_ERR_SHAPE, ("safetensors: unsupported dtype " + dt + " for " + name).c_str());
        if (b1 < b0 || b1 > data_len || b1 - b0 != count * esz)
            return fail(EBH_ERR_SHAPE, ("safetensors: bad data_offsets for " + name).c_str());
        raw.resize(b1 - b0);
        if (fseek(f.get(), (long)(data_start + b0), SEEK_SET) != 0 ||
            fread(raw.data(), 1, raw.size(), f.get()) != raw.size())
            return fail(EBH_ERR_SHAPE, ("safetensors: read failed for " + name).c_str());
        buf.resize(count);
        if (esz == 4) {
            memcpy(buf.data(), raw.data(), raw.size());  // little-endian host
        } else {
            for (uint64_t i = 0; i < count; ++i) {
                const uint16_t h = (uint16_t)(raw[2 * i] | (raw[2 * i + 1] << 8));
                buf[i] = dt == "F16" ? half_to_float(h) : bf16_to_float(h);
            }
        }
        const int rc = ebh_set_tensor(m, name.c_str(), buf.data(), shape.data(), (int32_t)shape.size());
        if (rc) return rc;
    }
    return EBH_OK;
}
