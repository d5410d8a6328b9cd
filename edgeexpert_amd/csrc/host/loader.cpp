// loader.cpp — tfq_loader.h: the packed-experts layout reader and the loaders
// that bring a repacked (.gturbo) checkpoint into device memory.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../../include/tfq_loader.h"
#include "json.hpp"
#include "module.hpp"

using tfq::fail;
using tfq::hip_check;
namespace json = tfq::json;

struct tfq_expert_layout {
    struct Tensor {
        uint64_t offset = 0, size = 0;
        std::string dtype;
        std::vector<int64_t> shape;
        bool has_bits = false;
        int64_t bits = 0;
    };
    struct Expert {
        int64_t expert = 0, physical_rank = 0;
        uint64_t offset = 0, size = 0;
        std::map<std::string, Tensor> tensors;
    };
    struct Layer {
        int64_t layer = 0;
        std::string file;
        std::vector<Expert> experts;
    };
    uint64_t expert_stride = 0;
    int64_t num_layers = 0, experts_per_layer = 0;
    std::vector<Layer> layers;
};

namespace {

constexpr uint64_t kDefaultLayoutCap = 16ull * 1024 * 1024;    // PackedExpertsLayout.swift:53

// (x as? NSNumber)?.uint64Value: any number, truncated / wrapped like the bridge.
bool number_u64(const json::Value* v, uint64_t& out) {
    if (!v || v->kind != json::Value::Number) return false;
    if (v->is_int) out = v->neg ? (uint64_t)(0 - v->u) : v->u;
    else out = (uint64_t)(int64_t)v->d;
    return true;
}
// x as? Int
bool as_int(const json::Value* v, int64_t& out) { return v && v->as_int(out); }

int corrupt(const char* detail) { return fail(TFQ_E_INVAL, "indexCorrupt: %s", detail); }

bool read_file(const std::string& path, std::string& out) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) return false;
    struct stat st {};
    if (::fstat(fd, &st) != 0) {
        ::close(fd);
        return false;
    }
    out.resize((size_t)st.st_size);
    size_t got = 0;
    while (got < out.size()) {
        const ssize_t n = ::pread(fd, &out[got], out.size() - got, (off_t)got);
        if (n <= 0) break;
        got += (size_t)n;
    }
    ::close(fd);
    return got == out.size();
}

// Reads exactly `size` bytes at `offset`; false on a short read or error.
bool pread_all(int fd, void* dst, uint64_t size, uint64_t offset) {
    uint64_t got = 0;
    while (got < size) {
        const ssize_t n = ::pread(fd, static_cast<char*>(dst) + got, size - got, (off_t)(offset + got));
        if (n <= 0) return false;
        got += (uint64_t)n;
    }
    return true;
}

// PackedExpertsLayoutReader.load (PackedExpertsLayout.swift:55-137).
int parse_layout(const std::string& text, tfq_expert_layout& L) {
    json::Value root;
    json::Parser parser(text.data(), text.size());
    if (!parser.parse(root)) {
        char msg[300];
        std::snprintf(msg, sizeof(msg), "layout.json: %s", parser.error().c_str());
        return corrupt(msg);
    }
    const json::Value* layers = root.get("layers");
    bool layers_ok = layers && layers->kind == json::Value::Array;
    if (layers_ok)
        for (const auto& l : layers->a) layers_ok = layers_ok && l.kind == json::Value::Object;
    if (!number_u64(root.get("expertStride"), L.expert_stride) || !as_int(root.get("numLayers"), L.num_layers) ||
        !as_int(root.get("expertsPerLayer"), L.experts_per_layer) || !layers_ok)
        return corrupt("layout.json: missing top-level keys");
    // the reference sizes an array by expertsPerLayer and traps on a negative count
    if (L.experts_per_layer < 0) return corrupt("layout.json: negative expertsPerLayer");
    const size_t E = (size_t)L.experts_per_layer;
    for (const json::Value& lo : layers->a) {
        tfq_expert_layout::Layer layer;
        const json::Value* file = lo.get("file");
        const json::Value* experts = lo.get("experts");
        bool experts_ok = experts && experts->kind == json::Value::Array;
        if (experts_ok)
            for (const auto& e : experts->a) experts_ok = experts_ok && e.kind == json::Value::Object;
        if (!as_int(lo.get("layer"), layer.layer) || !file || file->kind != json::Value::String || !experts_ok)
            return corrupt("layout.json: malformed layer entry");
        layer.file = file->s;
        std::vector<tfq_expert_layout::Expert> slots(E);
        std::vector<bool> filled(E, false);
        size_t placed = 0;
        for (const json::Value& eo : experts->a) {
            tfq_expert_layout::Expert ex;
            const json::Value* tensors = eo.get("tensors");
            bool tensors_ok = tensors && tensors->kind == json::Value::Object;
            if (tensors_ok)
                for (const auto& kv : tensors->o) tensors_ok = tensors_ok && kv.second.kind == json::Value::Object;
            if (!number_u64(eo.get("offset"), ex.offset) || !number_u64(eo.get("size"), ex.size) || !tensors_ok)
                return corrupt("layout.json: malformed expert entry");
            for (const auto& kv : tensors->o) {
                const json::Value& t = kv.second;
                tfq_expert_layout::Tensor tt;
                const json::Value* size = t.get("size");
                const json::Value* dtype = t.get("dtype");
                const json::Value* shape = t.get("shape");
                bool shape_ok = shape && shape->kind == json::Value::Array;
                if (shape_ok)
                    for (const auto& d : shape->a) {
                        int64_t dim;
                        shape_ok = shape_ok && as_int(&d, dim);
                        if (shape_ok) tt.shape.push_back(dim);
                    }
                if (!number_u64(t.get("offset"), tt.offset) || !size || size->kind != json::Value::Number ||
                    !dtype || dtype->kind != json::Value::String || !shape_ok) {
                    char msg[300];
                    std::snprintf(msg, sizeof(msg), "layout.json: malformed tensor %s", kv.first.c_str());
                    return corrupt(msg);
                }
                number_u64(size, tt.size);
                tt.dtype = dtype->s;
                if (const json::Value* bits = t.get("bits")) {
                    if (!as_int(bits, tt.bits)) {
                        char msg[300];
                        std::snprintf(msg, sizeof(msg), "layout.json: malformed tensor bits %s", kv.first.c_str());
                        return corrupt(msg);
                    }
                    tt.has_bits = true;
                }
                ex.tensors[kv.first] = tt;
            }
            int64_t id;
            if (!as_int(eo.get("expert"), id)) id = (int64_t)placed;     // entries placed so far
            if (id < 0 || id >= (int64_t)E) return corrupt("layout.json: expert id out of range");
            int64_t rank;
            if (!as_int(eo.get("physicalRank"), rank)) rank = id;
            if (rank < 0 || rank >= (int64_t)E) return corrupt("layout.json: physicalRank out of range");
            ex.expert = id;
            ex.physical_rank = rank;
            if (!filled[(size_t)id]) ++placed;
            filled[(size_t)id] = true;
            slots[(size_t)id] = ex;
        }
        if (placed != E) return corrupt("layout.json: missing expert entries");
        layer.experts = std::move(slots);
        L.layers.push_back(std::move(layer));
    }
    return TFQ_OK;
}

// The resident pool form of one expert blob (see tfq_expert_pool_load).
struct PoolForm {
    uint64_t wb = 0, sbg = 0, sbd = 0, blob = 0, stride = 0;
    tfq_expert_offsets off{};
};

bool pool_form(uint32_t d, uint32_t f, uint32_t bits, PoolForm& p) {
    if (d == 0 || f == 0 || d % TFQ_GROUP_SIZE || f % TFQ_GROUP_SIZE) return false;
    p.wb = (uint64_t)f * d / 8 * bits;
    p.sbg = (uint64_t)f * (d / 64) * 2;
    p.sbd = (uint64_t)d * (f / 64) * 2;
    p.blob = 3 * p.wb + 4 * p.sbg + 2 * p.sbd;
    p.stride = (p.blob + 255) / 256 * 256;
    if (p.blob > UINT32_MAX) return false;                  // offsets are 32-bit
    const uint64_t s0 = 3 * p.wb;
    p.off = {0u, (uint32_t)s0, (uint32_t)(s0 + p.sbg),
             (uint32_t)p.wb, (uint32_t)(s0 + 2 * p.sbg), (uint32_t)(s0 + 3 * p.sbg),
             (uint32_t)(2 * p.wb), (uint32_t)(s0 + 4 * p.sbg), (uint32_t)(s0 + 4 * p.sbg + p.sbd)};
    return true;
}

// One sub-tensor of a layer file's expert: where it is in the blob and where
// it goes in the pool form.
struct Part {
    const char* role;
    bool weights;
    uint64_t rows, cols;      // logical shape
    uint32_t dst;
    uint64_t bytes;
    uint64_t src = 0;
};

// Code width of a layer's routed experts: the `bits` of its first expert's
// gate weights (the repacker writes 4, TurboFieldfareRebits 2 or 3,
// Rebits/main.swift:437-441); 0 if absent or not 2..4 (check_part reports it).
uint32_t layer_bits(const tfq_expert_layout::Layer& l) {
    if (l.experts.empty()) return 0;
    auto it = l.experts[0].tensors.find("gate");
    if (it == l.experts[0].tensors.end() || !it->second.has_bits) return 0;
    const int64_t b = it->second.bits;
    return b >= 2 && b <= 4 ? (uint32_t)b : 0u;
}

// Every weight tensor must hold `bits`-bit codes (one width per pool).
int check_part(const tfq_expert_layout::Expert& ex, Part& p, uint32_t bits) {
    auto it = ex.tensors.find(p.role);
    if (it == ex.tensors.end())
        return fail(TFQ_E_INVAL, "expert %lld has no tensor %s", (long long)ex.expert, p.role);
    const tfq_expert_layout::Tensor& t = it->second;
    const bool shape_ok = p.weights ? (t.shape.size() == 2 && (uint64_t)t.shape[0] == p.rows &&
                                       (uint64_t)t.shape[1] == p.cols)
                                    : (t.shape.size() == 2 && (uint64_t)t.shape[0] == p.rows &&
                                       (uint64_t)t.shape[1] == p.cols / 64);
    if (p.weights && (t.dtype != "U32" || !t.has_bits || t.bits < 2 || t.bits > 4))
        return fail(TFQ_E_UNSUPPORTED, "expert %lld %s: %s weights of %lld bits (U32 of 2, 3 or 4 bits only)",
                    (long long)ex.expert, p.role, t.dtype.c_str(), (long long)t.bits);
    if (p.weights && (uint32_t)t.bits != bits)
        return fail(TFQ_E_UNSUPPORTED, "expert %lld %s: %lld-bit weights in a layer of %u-bit experts",
                    (long long)ex.expert, p.role, (long long)t.bits, bits);
    if (!p.weights && t.dtype != "BF16")
        return fail(TFQ_E_INVAL, "expert %lld %s: dtype %s, expected BF16", (long long)ex.expert, p.role,
                    t.dtype.c_str());
    if (!shape_ok || t.size != p.bytes)
        return fail(TFQ_E_INVAL, "expert %lld %s: shape/size do not match d, f", (long long)ex.expert, p.role);
    if (t.offset > ex.size || t.size > ex.size - t.offset)
        return fail(TFQ_E_INVAL, "expert %lld %s lies outside its blob", (long long)ex.expert, p.role);
    p.src = t.offset;
    return TFQ_OK;
}

// Pinned host staging buffer (hipHostMalloc), freed on scope exit.
struct Pinned {
    void* p = nullptr;
    ~Pinned() {
        if (p) (void)hipHostFree(p);
    }
};

// Waits for a stream's queued copies when leaving scope (declared after the
// staging buffer they read, so it runs before the buffer is freed).
struct StreamDrain {
    hipStream_t s = nullptr;
    bool armed = false;
    ~StreamDrain() {
        if (armed) (void)hipStreamSynchronize(s);
    }
};

struct Fd {
    int fd = -1;
    ~Fd() {
        if (fd >= 0) ::close(fd);
    }
};

}  // namespace

extern "C" {

int tfq_expert_layout_load(const char* model_dir, uint64_t max_bytes, tfq_expert_layout** out) {
    if (!model_dir || !out) return fail(TFQ_E_INVAL, "null pointer argument");
    *out = nullptr;
    const std::string path = std::string(model_dir) + "/packed_experts/layout.json";
    struct stat st {};
    if (::stat(path.c_str(), &st) != 0) return fail(TFQ_E_IO, "missingFile: packed_experts/layout.json");
    const uint64_t cap = max_bytes ? max_bytes : kDefaultLayoutCap;
    if ((uint64_t)st.st_size > cap) {
        char msg[200];
        std::snprintf(msg, sizeof(msg), "layout.json size %llu exceeds metadata cap %llu",
                      (unsigned long long)st.st_size, (unsigned long long)cap);
        return corrupt(msg);
    }
    std::string text;
    if (!read_file(path, text)) return fail(TFQ_E_IO, "cannot read packed_experts/layout.json: %s", std::strerror(errno));
    auto* L = new tfq_expert_layout();
    const int rc = parse_layout(text, *L);
    if (rc) {
        delete L;
        return rc;
    }
    *out = L;
    return TFQ_OK;
}

void tfq_expert_layout_free(tfq_expert_layout* layout) { delete layout; }

int tfq_expert_layout_info(const tfq_expert_layout* L, uint64_t* expert_stride, uint32_t* num_layers,
                           uint32_t* experts_per_layer, uint32_t* layer_entries) {
    if (!L) return fail(TFQ_E_INVAL, "null layout");
    if (expert_stride) *expert_stride = L->expert_stride;
    if (num_layers) *num_layers = (uint32_t)L->num_layers;
    if (experts_per_layer) *experts_per_layer = (uint32_t)L->experts_per_layer;
    if (layer_entries) *layer_entries = (uint32_t)L->layers.size();
    return TFQ_OK;
}

int tfq_expert_layout_expert(const tfq_expert_layout* L, uint32_t layer, uint32_t expert, uint32_t* physical_rank,
                             uint64_t* offset, uint64_t* size) {
    if (!L) return fail(TFQ_E_INVAL, "null layout");
    if (layer >= L->layers.size()) return fail(TFQ_E_INVAL, "layer %u of %zu", layer, L->layers.size());
    if (expert >= L->layers[layer].experts.size())
        return fail(TFQ_E_INVAL, "expert %u of %zu", expert, L->layers[layer].experts.size());
    const tfq_expert_layout::Expert& e = L->layers[layer].experts[expert];
    if (physical_rank) *physical_rank = (uint32_t)e.physical_rank;
    if (offset) *offset = e.offset;
    if (size) *size = e.size;
    return TFQ_OK;
}

int tfq_expert_layout_offsets(const tfq_expert_layout* L, uint32_t layer, tfq_expert_offsets* offsets, char* file,
                              size_t file_capacity) {
    if (!L || !offsets) return fail(TFQ_E_INVAL, "null pointer argument");
    if (layer >= L->layers.size()) return fail(TFQ_E_INVAL, "layer %u of %zu", layer, L->layers.size());
    const tfq_expert_layout::Layer& l = L->layers[layer];
    if (l.experts.empty()) return fail(TFQ_E_INVAL, "layer %u has no experts", layer);
    const auto& t = l.experts[0].tensors;
    auto off = [&](const char* role) -> uint32_t {
        auto it = t.find(role);
        return it == t.end() ? 0u : (uint32_t)it->second.offset;
    };
    *offsets = {off("gate"), off("gate_scales"), off("gate_biases"), off("up"),         off("up_scales"),
                off("up_biases"), off("down"), off("down_scales"), off("down_biases")};
    if (file && file_capacity) {
        std::strncpy(file, l.file.c_str(), file_capacity - 1);
        file[file_capacity - 1] = '\0';
    }
    return TFQ_OK;
}

int tfq_expert_pool_bytes(const tfq_expert_layout* L, uint32_t d, uint32_t f, uint64_t* stride, uint64_t* bytes) {
    if (!L) return fail(TFQ_E_INVAL, "null layout");
    // the widest layer sets the size (every layer's pool then fits)
    uint32_t bits = 2;
    for (const tfq_expert_layout::Layer& l : L->layers) bits = std::max(bits, layer_bits(l) ? layer_bits(l) : 4u);
    PoolForm p;
    if (!pool_form(d, f, bits, p)) return fail(TFQ_E_INVAL, "d=%u and f=%u must be positive multiples of 64", d, f);
    if (stride) *stride = p.stride;
    if (bytes) *bytes = p.stride * (uint64_t)L->experts_per_layer;
    return TFQ_OK;
}

int tfq_expert_pool_load(tfq_ctx* ctx, void* stream, const tfq_expert_layout* L, const char* model_dir,
                         uint32_t layer, uint32_t d, uint32_t f, void* pool, uint64_t pool_bytes,
                         tfq_expert_pool* desc, uint32_t* inexact_count_dev) {
    if (!ctx || !L || !model_dir || !pool || !desc) return fail(TFQ_E_INVAL, "null pointer argument");
    if (layer >= L->layers.size()) return fail(TFQ_E_INVAL, "layer %u of %zu", layer, L->layers.size());
    const tfq_expert_layout::Layer& l = L->layers[layer];
    const uint32_t bits = layer_bits(l) ? layer_bits(l) : 4u;      // a bad width fails in check_part
    PoolForm pf;
    if (!pool_form(d, f, bits, pf)) return fail(TFQ_E_INVAL, "d=%u and f=%u must be positive multiples of 64", d, f);
    if (!tfq::aligned(pool, 256)) return fail(TFQ_E_INVAL, "pool must be 256-byte aligned");
    const uint64_t E = l.experts.size();
    if (E == 0) return fail(TFQ_E_INVAL, "layer %u has no experts", layer);
    if (E > UINT32_MAX || pool_bytes < pf.stride * E) return fail(TFQ_E_INVAL, "pool smaller than %llu bytes",
                                                                   (unsigned long long)(pf.stride * E));
    // validate every expert before touching the device
    std::vector<std::vector<Part>> parts(E);
    uint64_t max_blob = 0;
    for (uint64_t e = 0; e < E; ++e) {
        const tfq_expert_layout::Expert& ex = l.experts[e];
        parts[e] = {{"gate", true, f, d, pf.off.gate_w, pf.wb},         {"up", true, f, d, pf.off.up_w, pf.wb},
                    {"down", true, d, f, pf.off.down_w, pf.wb},         {"gate_scales", false, f, d, pf.off.gate_s, pf.sbg},
                    {"gate_biases", false, f, d, pf.off.gate_b, pf.sbg}, {"up_scales", false, f, d, pf.off.up_s, pf.sbg},
                    {"up_biases", false, f, d, pf.off.up_b, pf.sbg},     {"down_scales", false, d, f, pf.off.down_s, pf.sbd},
                    {"down_biases", false, d, f, pf.off.down_b, pf.sbd}};
        for (Part& p : parts[e])
            if (int rc = check_part(ex, p, bits)) return rc;
        max_blob = std::max(max_blob, ex.size);
    }
    const std::string rel = "packed_experts/" + l.file;
    Fd fd;
    fd.fd = ::open((std::string(model_dir) + "/" + rel).c_str(), O_RDONLY);
    if (fd.fd < 0) return fail(TFQ_E_IO, "missingFile: %s", rel.c_str());
    // a few blobs per batch of reads; the device copies of a batch are queued
    // on `stream` and awaited before the staging is reused
    constexpr uint64_t kBatch = 8;
    Pinned staging;
    if (int rc = hip_check(hipHostMalloc(&staging.p, max_blob * kBatch, hipHostMallocDefault), "hipHostMalloc"))
        return rc;
    hipStream_t s = (hipStream_t)stream;
    StreamDrain drain{s, true};                 // error returns leave no copy reading freed staging
    char* dev = static_cast<char*>(pool);
    for (uint64_t e0 = 0; e0 < E; e0 += kBatch) {
        const uint64_t e1 = std::min(E, e0 + kBatch);
        for (uint64_t e = e0; e < e1; ++e) {
            const tfq_expert_layout::Expert& ex = l.experts[e];
            char* blob = static_cast<char*>(staging.p) + (e - e0) * max_blob;
            if (!pread_all(fd.fd, blob, ex.size, ex.offset))
                return fail(TFQ_E_IO, "%s: expert %llu (bytes %llu..%llu) past the end of the file", rel.c_str(),
                            (unsigned long long)e, (unsigned long long)ex.offset,
                            (unsigned long long)(ex.offset + ex.size));
            char* dst = dev + e * pf.stride;
            for (const Part& p : parts[e])
                if (int rc = hip_check(hipMemcpyAsync(dst + p.dst, blob + p.src, p.bytes, hipMemcpyHostToDevice, s),
                                       "hipMemcpyAsync"))
                    return rc;
            // the six BF16 scale/bias arrays are contiguous in the pool form
            auto* sb = reinterpret_cast<uint16_t*>(dst + pf.off.gate_s);
            if (int rc = tfq_convert_bf16_to_f16(ctx, stream, sb, sb, (4 * pf.sbg + 2 * pf.sbd) / 2, inexact_count_dev))
                return rc;
        }
        if (int rc = hip_check(hipStreamSynchronize(s), "hipStreamSynchronize")) return rc;
    }
    desc->base = pool;
    desc->stride = pf.stride;
    desc->num_experts = (uint32_t)E;
    desc->offsets = pf.off;
    desc->weight_bits = bits;
    return TFQ_OK;
}

int tfq_resident_load(void* stream, const char* path, uint64_t file_offset, uint64_t size, void* dst) {
    if (!path || (!dst && size)) return fail(TFQ_E_INVAL, "null pointer argument");
    Fd fd;
    fd.fd = ::open(path, O_RDONLY);
    if (fd.fd < 0) return fail(TFQ_E_IO, "missingFile: %s", path);
    struct stat st {};
    if (::fstat(fd.fd, &st) != 0 || file_offset > (uint64_t)st.st_size || size > (uint64_t)st.st_size - file_offset)
        return fail(TFQ_E_IO, "%s: bytes %llu..%llu past the end of the file", path, (unsigned long long)file_offset,
                    (unsigned long long)(file_offset + size));
    constexpr uint64_t kChunk = 64ull << 20;
    Pinned staging;
    if (size == 0) return TFQ_OK;
    if (int rc = hip_check(hipHostMalloc(&staging.p, std::min(size, kChunk), hipHostMallocDefault), "hipHostMalloc"))
        return rc;
    hipStream_t s = (hipStream_t)stream;
    for (uint64_t done = 0; done < size;) {
        const uint64_t n = std::min(kChunk, size - done);
        if (!pread_all(fd.fd, staging.p, n, file_offset + done))
            return fail(TFQ_E_IO, "%s: short read at %llu", path, (unsigned long long)(file_offset + done));
        if (int rc = hip_check(hipMemcpyAsync(static_cast<char*>(dst) + done, staging.p, n, hipMemcpyHostToDevice, s),
                               "hipMemcpyAsync"))
            return rc;
        if (int rc = hip_check(hipStreamSynchronize(s), "hipStreamSynchronize")) return rc;
        done += n;
    }
    return TFQ_OK;
}

}  // extern "C"
