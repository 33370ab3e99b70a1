// safetensors.cpp -- model.safetensors reader behind ebh_load_safetensors.
//
// Replaces ModelWeights::load (src/weights.rs:15-45).  File layout: an
// 8-byte little-endian header length N, N bytes of JSON mapping each tensor
// name to {"dtype", "shape", "data_offsets": [begin, end]} (offsets relative
// to the end of the header), optional "__metadata__", then the raw data.
// The reference decodes every tensor as f32 LE whatever its dtype
// (src/weights.rs:25-29).  Here the file is mapped, each tensor the encoder
// needs is handed to the model as a view of its bytes in the mapping (F32,
// F16 or BF16), and ebh_finalize uploads it from there in that encoding: no
// host copy, 16-bit tensors cross PCIe at 16 bits and are converted on the
// device (BF16 GEMM weights of bf16 models not at all).  Any other dtype of a
// needed tensor is an error; tensors the encoder does not use are skipped.
// The mapping is released at ebh_finalize or ebh_destroy, so the file must
// not be truncated before then.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

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

int fail(int code, const std::string& msg) { return ebh::set_error(code, "%s", msg.c_str()); }

// A read-only private mapping of the whole file, unmapped with its last owner.
std::shared_ptr<const void> map_file(const char* path, size_t* size, std::string* err) {
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        *err = std::string("cannot open ") + path;
        return nullptr;
    }
    struct stat sb;
    if (fstat(fd, &sb) != 0 || !S_ISREG(sb.st_mode)) {
        close(fd);
        *err = std::string("cannot open ") + path + " (not a regular file)";
        return nullptr;
    }
    *size = (size_t)sb.st_size;
    if (*size < 8) {
        close(fd);
        *err = "safetensors: truncated header";
        return nullptr;
    }
    void* p = mmap(nullptr, *size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (p == MAP_FAILED) {
        *err = std::string("cannot map ") + path;
        return nullptr;
    }
    const size_t n = *size;
    return std::shared_ptr<const void>(p, [n](const void* q) { munmap(const_cast<void*>(q), n); });
}

}  // namespace

extern "C" int ebh_load_safetensors(ebh_model* m, const char* path) {
    if (!m || !path) return fail(EBH_ERR_INVALID_ARG, "null argument");
    size_t fsize = 0;
    std::string err;
    std::shared_ptr<const void> map = map_file(path, &fsize, &err);
    if (!map) return fail(err.rfind("cannot", 0) == 0 ? EBH_ERR_NOT_FOUND : EBH_ERR_SHAPE, err);
    const uint8_t* bytes = static_cast<const uint8_t*>(map.get());
    uint64_t n = 0;
    for (int i = 7; i >= 0; --i) n = (n << 8) | bytes[i];
    if (n > (100u << 20)) return fail(EBH_ERR_SHAPE, "safetensors: header too large");
    if (n > fsize - 8) return fail(EBH_ERR_SHAPE, "safetensors: truncated header");
    const uint64_t data_start = 8 + n;
    const uint64_t data_len = (uint64_t)fsize - data_start;
    const char* header = reinterpret_cast<const char*>(bytes + 8);

    Parser ps{header, header + n, {}};
    JVal root;
    if (!ps.parse(root) || root.kind != JVal::OBJ)
        return fail(EBH_ERR_SHAPE, "safetensors: bad header JSON: " + ps.err);

    for (auto& kv : root.obj) {
        const std::string& name = kv.first;
        if (name == "__metadata__") continue;
        const JVal& t = kv.second;
        if (t.kind != JVal::OBJ || !t.obj.count("dtype") || !t.obj.count("shape") || !t.obj.count("data_offsets"))
            return fail(EBH_ERR_SHAPE, "safetensors: malformed entry " + name);
        // The encoder's tensors and the cross-encoder head; pooler / position_ids are skipped.
        const bool wanted = name.rfind("embeddings.", 0) == 0 || name.rfind("encoder.layer.", 0) == 0 ||
                            name == "classifier.weight" || name == "classifier.bias";
        if (!wanted || name == "embeddings.position_ids") continue;
        const std::string& dt = t.obj.at("dtype").str;
        const JVal& shp = t.obj.at("shape");
        const JVal& offs = t.obj.at("data_offsets");
        if (shp.kind != JVal::ARR || offs.kind != JVal::ARR || offs.arr.size() != 2)
            return fail(EBH_ERR_SHAPE, "safetensors: malformed entry " + name);
        std::vector<int64_t> shape;
        uint64_t count = 1;
        for (auto& d : shp.arr) {
            // Dimensions are non-negative integers; 2^40 bounds the element
            // count of any tensor this model could hold.
            if (d.kind != JVal::NUM || !(d.num >= 0.0) || d.num != (double)(int64_t)d.num ||
                d.num > (double)(1ull << 40))
                return fail(EBH_ERR_SHAPE, "safetensors: bad shape for " + name);
            shape.push_back((int64_t)d.num);
            count *= (uint64_t)d.num;
            if (count > (1ull << 40)) return fail(EBH_ERR_SHAPE, "safetensors: bad shape for " + name);
        }
        for (auto& o : offs.arr)
            if (o.kind != JVal::NUM || !(o.num >= 0.0) || o.num > 9.0e15)
                return fail(EBH_ERR_SHAPE, "safetensors: bad data_offsets for " + name);
        const uint64_t b0 = (uint64_t)offs.arr[0].num, b1 = (uint64_t)offs.arr[1].num;
        // The reference reads every tensor as f32 LE (src/weights.rs:25-29);
        // here F16 and BF16 stay 16-bit until the device converts them.
        const int kind = dt == "F32" ? ebh::TENSOR_F32 : dt == "F16" ? ebh::TENSOR_F16
                       : dt == "BF16" ? ebh::TENSOR_BF16 : -1;
        if (kind < 0) return fail(EBH_ERR_SHAPE, "safetensors: unsupported dtype " + dt + " for " + name);
        const uint64_t esz = kind == ebh::TENSOR_F32 ? 4 : 2;
        if (b1 < b0 || b1 > data_len || b1 - b0 != count * esz)
            return fail(EBH_ERR_SHAPE, "safetensors: bad data_offsets for " + name);
        const int rc = ebh::put_tensor(m, name.c_str(), bytes + data_start + b0, kind, shape.data(),
                                       (int32_t)shape.size(), map);
        if (rc) return rc;
    }
    return EBH_OK;
}
