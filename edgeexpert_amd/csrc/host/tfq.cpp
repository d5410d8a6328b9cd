// tfq.cpp — libtfq: the C ABI of include/tfq.h and include/tfq_runtime.h.
//
// Loads the gfx950 code object (hipModuleLoad), resolves every kernel once
// (hipModuleGetFunction), and forwards each C entry point to the operator
// class that mirrors the reference wrapper (ops.hpp). No entry point
// allocates device memory or synchronises the caller's stream.
#include <dlfcn.h>
#include <sys/stat.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "../../../include/tfq_runtime.h"
#include "noalloc.hpp"
#include "ops.hpp"

namespace tfq {

ErrorState& error_state() {
    static thread_local ErrorState s;
    return s;
}

static std::vector<std::string> kernel_names() {
    std::vector<std::string> names;
    const char* q4_shapes[] = {"s2_p1",  "s4_p1",  "s8_p1",  "s8_p2",  "s8_p3",  "s8_p4",
                               "s16_p1", "s16_p2", "s16_p3", "s16_p4", "s32_p1", "s32_p2",
                               "s32_p3", "s32_p4", "s64_p1", "s64_p2", "s64_p3", "s64_p4"};
    const char* q8_shapes[] = {"s4_p1", "s8_p1", "s16_p1", "s32_p1",
                               "s64_p1", "s64_p2", "s64_p3", "s64_p4"};
    for (const char* s : q4_shapes)
        for (const char* form : {"", "norm_"}) {
            names.push_back(std::string("tfq_q4_gemv_") + form + s);
            if (*form) {
                names.push_back(std::string("tfq_q4_gemv_tail_") + s);
                names.push_back(std::string("tfq_q4_gemv_rms_") + s);
                names.push_back(std::string("tfq_q4_gemv_wide_") + s);
                names.push_back(std::string("tfq_q3_gemv_rms_") + s);
            }
            names.push_back(std::string("tfq_q3_gemv_") + form + s);
            for (const char* b : {"", "b2_", "b3_"}) {
                names.push_back(std::string("tfq_moe_phase1_") + b + form + s);
                names.push_back(std::string("tfq_moe_phase1_routed_") + b + form + s);
            }
            if (*form) {
                names.push_back(std::string("tfq_moe_phase1_shared_") + s);
                names.push_back(std::string("tfq_gate_up_act_c_") + s);
            }
            names.push_back(std::string("tfq_gate_up_act_") + form + s);
        }
    for (const char* s : q4_shapes) {
        names.push_back(std::string("tfq_lm_head_greedy_") + s);
        names.push_back(std::string("tfq_lm_head_greedy_rms_") + s);
    }
    names.push_back("tfq_lm_head_reduce");
    for (const char* s : q8_shapes) {
        names.push_back(std::string("tfq_q8_gemv_") + s);
        names.push_back(std::string("tfq_q8_gemv_c_") + s);
        names.push_back(std::string("tfq_q8_gate_up_act_") + s);
        names.push_back(std::string("tfq_q8_gate_up_act_c_") + s);
        names.push_back(std::string("tfq_q8_gate_up_act_norm_") + s);
        names.push_back(std::string("tfq_router_logits_") + s);
        names.push_back(std::string("tfq_router_logits_c_") + s);
        names.push_back(std::string("tfq_router_logits_pa_") + s);
        names.push_back(std::string("tfq_prefill_router_logits_") + s);
    }
    for (int p = 1; p <= 4; ++p) {
        for (const char* b : {"", "b2_", "b3_"}) names.push_back(std::string("tfq_moe_phase2_") + b + "p" + std::to_string(p));
        for (int sp = 1; sp <= 4; ++sp)
            names.push_back("tfq_moe_phase2_shared_p" + std::to_string(p) + "_sp" + std::to_string(sp));
        for (const char* q : {"4_1", "8_1", "16_1", "32_1", "64_1", "64_2", "64_3", "64_4"})
            names.push_back("tfq_moe_phase2_shared8_p" + std::to_string(p) + "_q" + q);
    }
    for (const char* n : {"s2_p1_q4_1", "s4_p1_q8_1", "s8_p1_q16_1", "s8_p3_q64_1", "s16_p1_q32_1", "s16_p3_q64_2",
                          "s32_p1_q64_1", "s32_p3_q64_3", "s64_p1_q64_2", "s64_p2_q64_4"})
        names.push_back(std::string("tfq_moe_phase1_shared8_") + n);
    names.push_back("tfq_router_select");
    names.push_back("tfq_read_ceiling");
    names.push_back("tfq_gelu_mul_f16");
    for (const char* n : {"tfq_gemm_q4_f16", "tfq_gemm_q4_bf16", "tfq_gemm_q3_f16", "tfq_gemm_q3_bf16"})
        names.push_back(n);
    for (const char* b : {"q4", "q3"})
        for (const char* dt : {"f16", "bf16"})
            for (const char* rt : {"r1", "r2"})
                for (int c = 1; c <= 8; ++c)
                    names.push_back(std::string("tfq_gemm_skinny_") + b + "_" + dt + "_" + rt + "_c" +
                                    std::to_string(c));
    for (const char* n : {"tfq_prefill_select", "tfq_moe_group", "tfq_moe_grouped_gate_up", "tfq_moe_grouped_down",
                          "tfq_moe_grouped_gate_up_b2", "tfq_moe_grouped_down_b2", "tfq_moe_grouped_gate_up_b3",
                          "tfq_moe_grouped_down_b3", "tfq_moe_grouped_gate_up_t", "tfq_moe_grouped_down_t",
                          "tfq_moe_grouped_gate_up_b2_t", "tfq_moe_grouped_down_b2_t", "tfq_moe_grouped_gate_up_b3_t",
                          "tfq_moe_grouped_down_b3_t", "tfq_moe_combine", "tfq_moe_combine_x8"})
        names.push_back(n);
    names.push_back("tfq_convert_bf16_f16");
    for (const char* hd : {"128", "256", "512"}) {
        for (const char* g : {"1", "2", "4"})
            names.push_back(std::string("tfq_attn_partial_h") + hd + "_g" + g);
        names.push_back(std::string("tfq_attn_combine_h") + hd);
    }
    names.push_back("tfq_attn_partial_h512_g8");
    names.push_back("tfq_layer_tail");
    return names;
}

// The code objects edgeexpert_amd/build.py writes next to libtfq.so.
static const char* const kCodeObjects[] = {"tfq_gemv", "tfq_int8",    "tfq_phase1",    "tfq_phase1_routed",
                                           "tfq_moe",  "tfq_gemm",    "tfq_prefill",   "tfq_attention",
                                           "tfq_layer_moe"};

int Module::load(const std::string& dir) {
    int rc = hip_check(hipGetDevice(&device_), "hipGetDevice");
    if (rc) return rc;
    int cus = 0;
    rc = hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device_),
                   "hipDeviceGetAttribute(multiProcessorCount)");
    if (rc) return rc;
    cus_ = cus > 0 ? (uint32_t)cus : 1u;
    for (const char* unit : kCodeObjects) {
        const std::string path = dir + "/" + unit + ".co";
        hipModule_t m = nullptr;
        rc = hip_check(hipModuleLoad(&m, path.c_str()), "hipModuleLoad");
        if (rc) return fail(rc, "hipModuleLoad(%s): %s", path.c_str(), error_state().message);
        modules_.push_back(m);
    }
    for (const std::string& n : kernel_names()) {
        hipFunction_t f = nullptr;
        for (hipModule_t m : modules_)
            if (hipModuleGetFunction(&f, m, n.c_str()) == hipSuccess && f) break;
        if (!f) return fail(TFQ_E_NOT_LOADED, "kernel %s missing from the code objects in %s", n.c_str(), dir.c_str());
        fns_[n] = f;
    }
    (void)hipGetLastError();     // the lookups above leave a not-found status behind
    return TFQ_OK;
}

uint32_t Module::resident_blocks(hipFunction_t f, uint32_t block, uint32_t lds) const {
    const auto key = std::make_pair(f, ((uint64_t)block << 32) | lds);
    std::lock_guard<std::mutex> lock(occ_mu_);
    auto it = occ_.find(key);
    if (it != occ_.end()) return it->second;
    int per_cu = 0;
    if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, (int)block, lds) != hipSuccess ||
        per_cu < 1)
        per_cu = 1;
    const uint32_t total = (uint32_t)per_cu * cus_;
    occ_.emplace(key, total);
    return total;
}

Module::~Module() {
    for (hipModule_t m : modules_) (void)hipModuleUnload(m);
}

// The directory of libtfq.so.
static std::string library_dir() {
    Dl_info info{};
    if (dladdr(reinterpret_cast<void*>(&library_dir), &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        size_t slash = p.rfind('/');
        return slash == std::string::npos ? std::string(".") : p.substr(0, slash);
    }
    return ".";
}

// A directory is used as is; a file path names the directory holding it.
static std::string code_object_dir(const char* path) {
    if (!path) return library_dir();
    struct stat st {};
    std::string p(path);
    if (stat(path, &st) == 0 && S_ISDIR(st.st_mode)) return p;
    size_t slash = p.rfind('/');
    return slash == std::string::npos ? std::string(".") : p.substr(0, slash);
}

}  // namespace tfq

using namespace tfq;

struct tfq_ctx {
    Module module;
    DequantInt4GEMV* int4 = nullptr;
    DequantInt8GEMV* int8 = nullptr;
    MoE* moe = nullptr;
    SharedExpertInt4* shared = nullptr;
    SharedExpertInt8* shared8 = nullptr;
    PrefillInt4QMM* qmm = nullptr;
    PrefillSharedExpert* pshared = nullptr;
    PrefillRouter* prouter = nullptr;
    PrefillMoEGrouping* grouping = nullptr;
    PrefillGroupedRoutedMoE* grouped = nullptr;
    Attention* attn = nullptr;
    DecodeLayer* layer = nullptr;
    LMHeadGreedyInt4* lmhead = nullptr;
    void* scratch = nullptr;           // this device's copy of the noalloc scratch array
    int scratch_status = TFQ_OK;       // hipGetSymbolAddress's outcome at creation
    char scratch_error[256] = {0};
    ~tfq_ctx() {
        delete lmhead;
        delete layer;
        delete pshared;
        delete shared8;
        delete attn;
        delete qmm;
        delete prouter;
        delete grouping;
        delete grouped;
        delete int4;
        delete int8;
        delete moe;
        delete shared;
    }
};

#define TFQ_REQUIRE_CTX(ctx) \
    if (!(ctx)) return fail(TFQ_E_INVAL, "null context")

extern "C" {

int tfq_create(tfq_ctx** out, const char* code_object_path) {
    if (!out) return fail(TFQ_E_INVAL, "null output pointer");
    *out = nullptr;
    tfq_ctx* c = new (std::nothrow) tfq_ctx();
    if (!c) return fail(TFQ_E_INVAL, "out of host memory");
    int rc = c->module.load(code_object_dir(code_object_path));
    if (rc) {
        delete c;
        return rc;
    }
    c->int4 = new DequantInt4GEMV(c->module);
    c->lmhead = new LMHeadGreedyInt4(c->module);
    c->int8 = new DequantInt8GEMV(c->module);
    c->moe = new MoE(c->module);
    c->shared = new SharedExpertInt4(c->module);
    c->shared8 = new SharedExpertInt8(c->module);
    c->qmm = new PrefillInt4QMM(c->module);
    c->pshared = new PrefillSharedExpert(c->module, *c->shared8, *c->qmm);
    c->prouter = new PrefillRouter(c->module);
    c->grouping = new PrefillMoEGrouping(c->module);
    c->grouped = new PrefillGroupedRoutedMoE(c->module);
    c->attn = new Attention(c->module);
    c->layer = new DecodeLayer(c->module, *c->int4, *c->moe, *c->shared, *c->shared8, *c->attn);
    // the allocation-free entry point's scratch on this device; a failure is
    // reported by that entry point, not by the context
    c->scratch_status = noalloc_scratch_address(&c->scratch);
    if (c->scratch_status != TFQ_OK) {
        std::snprintf(c->scratch_error, sizeof(c->scratch_error), "%s", error_state().message);
        c->scratch = nullptr;
    }
    *out = c;
    return TFQ_OK;
}

void tfq_destroy(tfq_ctx* ctx) { delete ctx; }

const char* tfq_status_string(int status) {
    switch (status) {
        case TFQ_OK: return "ok";
        case TFQ_E_INVAL: return "invalid argument (shape, alignment or null pointer)";
        case TFQ_E_UNSUPPORTED: return "shape not compiled into the code object";
        case TFQ_E_HIP: return "HIP runtime error";
        case TFQ_E_NOT_LOADED: return "kernel not loaded";
        case TFQ_E_IO: return "checkpoint file missing, unreadable or short";
        default: return "unknown status";
    }
}

int tfq_last_hip_error(void) { return error_state().hip; }
const char* tfq_last_error_message(void) { return error_state().message; }

int tfq_gemv_q4g64(tfq_ctx* ctx, void* stream, const void* weights, const uint16_t* scales,
                   const uint16_t* biases, const uint16_t* x, uint16_t* y, uint32_t m, uint32_t n) {
    TFQ_REQUIRE_CTX(ctx);
    return ctx->int4->encode(stream, weights, scales, biases, x, y, m, n);
}

int tfq_gemv_q4g64_qkv(tfq_ctx* ctx, void* stream, const tfq_q4_matrix* q, const tfq_q4_matrix* k,
                       const tfq_q4_matrix* v, const uint16_t* x, uint16_t* yq, uint16_t* yk,
                       uint16_t* yv, uint32_t mq, uint32_t mkv, uint32_t n) {
    TFQ_REQUIRE_CTX(ctx);
    if (!q || !k || !v) return fail(TFQ_E_INVAL, "null matrix descriptor");
    return ctx->int4->encode_qkv(stream, *q, *k, *v, x, yq, yk, yv, mq, mkv, n);
}

int tfq_gemv_qg64(tfq_ctx* ctx, void* stream, const void* weights, const uint16_t* scales,
                  const uint16_t* biases, const uint16_t* x, uint16_t* y, uint32_t m, uint32_t n, uint32_t bits) {
    TFQ_REQUIRE_CTX(ctx);
    return ctx->int4->encode(stream, weights, scales, biases, x, y, m, n, nullptr, stage_copy(), bits);
}

int tfq_gemv_qg64_qkv(tfq_ctx* ctx, void* stream, const tfq_q4_matrix* q, const tfq_q4_matrix* k,
                      const tfq_q4_matrix* v, const uint16_t* x, uint16_t* yq, uint16_t* yk, uint16_t* yv,
                      uint32_t mq, uint32_t mkv, uint32_t n, uint32_t bits) {
    TFQ_REQUIRE_CTX(ctx);
    if (!q || !k || !v) return fail(TFQ_E_INVAL, "null matrix descriptor");
    return ctx->int4->encode_qkv(stream, *q, *k, *v, x, yq, yk, yv, mq, mkv, n, stage_copy(), bits);
}

int tfq_lm_head_greedy(tfq_ctx* ctx, void* stream, const uint16_t* hidden, const uint16_t* norm_weight,
                       const void* weights, const uint16_t* scales, const uint16_t* biases, uint32_t* out_token,
                       uint32_t d, uint32_t vocab, float eps, void* workspace) {
    TFQ_REQUIRE_CTX(ctx);
    return ctx->lmhead->encode(stream, hidden, norm_weight, weights, scales, biases, out_token, d, vocab, eps,
                               workspace, TFQ_LM_HEAD_WORKSPACE_BYTES);
}

int tfq_gemv_q8g64(tfq_ctx* ctx, void* stream, const uint8_t* weights, const uint16_t* scales,
                   const uint16_t* biases, const uint16_t* x, uint16_t* y, uint32_t m, uint32_t n) {
    TFQ_REQUIRE_CTX(ctx);
    return ctx->int8->encode(stream, weights, scales, biases, x, y, m, n);
}

int tfq_router_topk(tfq_ctx* ctx, void* stream, const uint8_t* weights, const uint16_t* scales,
                    const uint16_t* biases, const uint16_t* hidden, const uint16_t* effective_scale,
                    const uint16_t* per_expert_scale, uint32_t* out_indices, uint16_t* out_weights,
                    float* out_weights_f32, float* out_logits_f32, uint32_t num_experts, uint32_t d,
                    uint32_t top_k, void* workspace) {
    TFQ_REQUIRE_CTX(ctx);
    return ctx->moe->encode_router_gemma4(stream, weights, scales, biases, hidden, effective_scale,
                                          per_expert_scale, out_indices, out_weights,
                                          out_weights_f32, out_logits_f32, num_experts, d, top_k,
                                          workspace);
}

int tfq_moe_phase1(tfq_ctx* ctx, void* stream, const tfq_expert_pool* pool, const uint32_t* indices,
                   const uint16_t* x, uint16_t* acts, uint32_t d, uint32_t f, uint32_t top_k) {
    TFQ_REQUIRE_CTX(ctx);
    if (!pool) return fail(TFQ_E_INVAL, "null pool");
    return ctx->moe->encode_phase1(stream, *pool, indices, x, acts, nullptr, top_k, d, f, top_k);
}

int tfq_moe_phase1_subset(tfq_ctx* ctx, void* stream, const tfq_expert_pool* pool,
                          const uint32_t* indices, const uint16_t* x, uint16_t* acts,
                          const uint32_t* active_slots, uint32_t active_count, uint32_t d,
                          uint32_t f, uint32_t top_k) {
    TFQ_REQUIRE_CTX(ctx);
    if (!pool) return fail(TFQ_E_INVAL, "null pool");
    if (!active_slots && active_count) return fail(TFQ_E_INVAL, "null active slot list");
    return ctx->moe->encode_phase1(stream, *pool, indices, x, acts, active_slots, active_count, d,
                                   f, top_k);
}

int tfq_moe_phase2(tfq_ctx* ctx, void* stream, const tfq_expert_pool* pool, const uint32_t* indices,
                   const uint16_t* acts, const uint16_t* routing_weights, const uint16_t* residual,
                   uint16_t* y, uint32_t d, uint32_t f, uint32_t top_k) {
    TFQ_REQUIRE_CTX(ctx);
    if (!pool) return fail(TFQ_E_INVAL, "null pool");
    return ctx->moe->encode_phase2(stream, *pool, indices, acts, routing_weights, residual, y, d, f,
                                   top_k);
}

int tfq_moe_decode(tfq_ctx* ctx, void* stream, const tfq_expert_pool* pool, const uint32_t* indices,
                   const uint16_t* routing_weights, const uint16_t* x, const uint16_t* residual,
                   uint16_t* y, uint32_t d, uint32_t f, uint32_t top_k, uint16_t* acts_scratch) {
    TFQ_REQUIRE_CTX(ctx);
    if (!pool) return fail(TFQ_E_INVAL, "null pool");
    int rc = ctx->moe->encode_phase1(stream, *pool, indices, x, acts_scratch, nullptr, top_k, d, f,
                                     top_k);
    if (rc) return rc;
    return ctx->moe->encode_phase2(stream, *pool, indices, acts_scratch, routing_weights, residual,
                                   y, d, f, top_k);
}

int tfq_router_logits(tfq_ctx* ctx, void* stream, const uint8_t* weights, const uint16_t* scales,
                      const uint16_t* biases, const uint16_t* hidden, const uint16_t* effective_scale,
                      float* logits, uint32_t num_experts, uint32_t d) {
    TFQ_REQUIRE_CTX(ctx);
    if (!logits) return fail(TFQ_E_INVAL, "null logits");
    float* used = nullptr;
    return ctx->moe->encode_router_logits(stream, weights, scales, biases, hidden, effective_scale, logits,
                                          num_experts, d, 1, logits, stage_copy(), &used);
}

int tfq_moe_phase1_routed(tfq_ctx* ctx, void* stream, const tfq_expert_pool* pool, const float* logits,
                          const uint16_t* per_expert_scale, uint32_t num_experts, uint32_t* out_indices,
                          uint16_t* out_weights, float* out_weights_f32, const uint16_t* x, uint16_t* acts,
                          uint32_t d, uint32_t f, uint32_t top_k) {
    TFQ_REQUIRE_CTX(ctx);
    if (!pool) return fail(TFQ_E_INVAL, "null pool");
    return ctx->moe->encode_phase1_routed(stream, *pool, logits, per_expert_scale, num_experts, out_indices,
                                          out_weights, out_weights_f32, x, acts, d, f, top_k);
}

int tfq_moe_decode_token(tfq_ctx* ctx, void* stream, const tfq_router* router,
                         const tfq_expert_pool* pool, const uint16_t* x, const uint16_t* residual,
                         uint16_t* y, uint32_t d, uint32_t f, uint32_t top_k, uint32_t* out_indices,
                         uint16_t* out_weights, uint16_t* acts_scratch, void* workspace) {
    TFQ_REQUIRE_CTX(ctx);
    if (!router || !pool) return fail(TFQ_E_INVAL, "null router or pool");
    if (router->num_experts != pool->num_experts)
        return fail(TFQ_E_INVAL, "router has %u experts, pool %u", router->num_experts,
                    pool->num_experts);
    float* logits = nullptr;
    int rc = ctx->moe->encode_router_logits(stream, router->weights, router->scales, router->biases, x,
                                            router->effective_scale, nullptr, router->num_experts, d, top_k,
                                            workspace, stage_copy(), &logits);
    if (rc) return rc;
    rc = ctx->moe->encode_phase1_routed(stream, *pool, logits, router->per_expert_scale, router->num_experts,
                                        out_indices, out_weights, nullptr, x, acts_scratch, d, f, top_k);
    if (rc) return rc;
    return ctx->moe->encode_phase2(stream, *pool, out_indices, acts_scratch, out_weights, residual,
                                   y, d, f, top_k);
}

int tfq_moe_decode_token_noalloc(tfq_ctx* ctx, void* stream, const tfq_router* router,
                                 const tfq_expert_pool* pool, const uint16_t* x, const uint16_t* residual,
                                 uint16_t* y, uint32_t d, uint32_t f, uint32_t top_k, uint32_t* out_indices,
                                 uint16_t* out_weights) {
    TFQ_REQUIRE_CTX(ctx);
    if (!ctx->scratch)
        return fail(ctx->scratch_status ? ctx->scratch_status : TFQ_E_HIP, "noalloc scratch unavailable: %s",
                    ctx->scratch_error);
    if ((uint64_t)top_k * f * 2 > kNoAllocActsBytes)
        return fail(TFQ_E_INVAL, "top_k * f * 2 = %llu bytes exceeds the %zu-byte scratch of the allocation-free "
                    "entry point", (unsigned long long)top_k * f * 2, kNoAllocActsBytes);
    uint8_t* base = static_cast<uint8_t*>(ctx->scratch);
    return tfq_moe_decode_token(ctx, stream, router, pool, x, residual, y, d, f, top_k, out_indices, out_weights,
                                reinterpret_cast<uint16_t*>(base), base + kNoAllocLogitsOffset);
}

int tfq_shared_expert_q4(tfq_ctx* ctx, void* stream, const tfq_q4_matrix* gate,
                         const tfq_q4_matrix* up, const tfq_q4_matrix* down, const uint16_t* x,
                         uint16_t* y, uint32_t d, uint32_t f, uint16_t* act_scratch) {
    TFQ_REQUIRE_CTX(ctx);
    if (!gate || !up || !down) return fail(TFQ_E_INVAL, "null matrix descriptor");
    return ctx->shared->encode(stream, x, *gate, *up, *down, y, d, f, act_scratch);
}

int tfq_shared_expert_q8(tfq_ctx* ctx, void* stream, const tfq_q8_matrix* gate, const tfq_q8_matrix* up,
                         const tfq_q8_matrix* down, const uint16_t* x, uint16_t* y, uint32_t d, uint32_t f,
                         uint16_t* act_scratch) {
    TFQ_REQUIRE_CTX(ctx);
    if (!gate || !up || !down) return fail(TFQ_E_INVAL, "null matrix descriptor");
    return ctx->shared8->encode(stream, x, *gate, *up, *down, y, d, f, act_scratch);
}

size_t tfq_prefill_shared_expert_workspace_bytes(uint32_t weight_bits, uint32_t tokens, uint32_t f) {
    return PrefillSharedExpert::workspace_bytes(weight_bits, tokens, f);
}

int tfq_prefill_shared_expert(tfq_ctx* ctx, void* stream, uint32_t weight_bits, const tfq_q4_matrix* gate,
                              const tfq_q4_matrix* up, const tfq_q4_matrix* down, const uint16_t* x,
                              uint32_t x_stride, uint16_t* y, uint32_t y_stride, uint32_t tokens, uint32_t d,
                              uint32_t f, void* workspace, size_t workspace_bytes) {
    TFQ_REQUIRE_CTX(ctx);
    if (!gate || !up || !down) return fail(TFQ_E_INVAL, "null matrix descriptor");
    return ctx->pshared->encode(stream, weight_bits, *gate, *up, *down, x, x_stride, y, y_stride, tokens, d, f,
                                workspace, workspace_bytes);
}

size_t tfq_attention_workspace_bytes(uint32_t head_dim, uint32_t num_q_heads, uint32_t seq_len,
                                     uint32_t window) {
    return Attention::workspace_bytes(head_dim, num_q_heads, seq_len, window);
}

int tfq_attention_decode(tfq_ctx* ctx, void* stream, const uint16_t* q, const uint16_t* k_cache,
                         const uint16_t* v_cache, uint16_t* out, uint32_t head_dim,
                         uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t seq_len,
                         uint32_t window, float scale, void* workspace, size_t workspace_bytes) {
    TFQ_REQUIRE_CTX(ctx);
    const AttnEpilogue none{nullptr, nullptr, 0.0f, 0.0f, 0, 0, 0.0, nullptr, nullptr};
    // without the epilogue the kernels only read the caches
    return ctx->attn->encode(stream, q, const_cast<uint16_t*>(k_cache), const_cast<uint16_t*>(v_cache),
                             out, head_dim, num_q_heads, num_kv_heads, seq_len, window, scale, none,
                             workspace, workspace_bytes);
}

size_t tfq_decode_layer_workspace_bytes(const tfq_decode_layer_shape* shape, uint32_t max_seq_len) {
    if (!shape || max_seq_len == 0) return 0;
    return DecodeLayer::layout(*shape, max_seq_len).total;
}

int tfq_abi_version(void) { return TFQ_ABI_VERSION; }

int tfq_decode_layer(tfq_ctx* ctx, void* stream, const tfq_decode_layer_weights* weights,
                     const tfq_decode_layer_shape* shape, const uint16_t* hidden_in,
                     uint16_t* hidden_out, uint16_t* k_cache, uint16_t* v_cache, uint32_t position,
                     uint32_t* out_indices, uint16_t* out_weights, void* workspace,
                     size_t workspace_bytes) {
    TFQ_REQUIRE_CTX(ctx);
    if (!weights || !shape) return fail(TFQ_E_INVAL, "null weights or shape");
    return ctx->layer->encode(stream, *weights, *shape, hidden_in, hidden_out, k_cache, v_cache, position,
                              out_indices, out_weights, workspace, workspace_bytes);
}

size_t tfq_decode_layers_workspace_bytes(const tfq_decode_layer_shape* shapes, uint32_t n_layers,
                                         uint32_t max_seq_len) {
    if (!shapes || n_layers == 0 || max_seq_len == 0) return 0;
    return DecodeLayer::chain_workspace_bytes(n_layers, shapes, max_seq_len);
}

int tfq_decode_layers(tfq_ctx* ctx, void* stream, uint32_t n_layers, const tfq_decode_layer_weights* weights,
                      const tfq_decode_layer_shape* shapes, const uint16_t* hidden_in, uint16_t* hiddens,
                      uint16_t* const* k_caches, uint16_t* const* v_caches, uint32_t position, void* workspace,
                      size_t workspace_bytes) {
    TFQ_REQUIRE_CTX(ctx);
    return ctx->layer->encode_chain(stream, n_layers, weights, shapes, hidden_in, hiddens, k_caches, v_caches,
                                    position, workspace, workspace_bytes);
}

int tfq_gemm_q4g64(tfq_ctx* ctx, void* stream, const void* weights, const uint16_t* scales,
                   const uint16_t* biases, const uint16_t* x, uint16_t* y, uint32_t m, uint32_t n,
                   uint32_t k, int dtype) {
    TFQ_REQUIRE_CTX(ctx);
    return ctx->qmm->encode(stream, weights, scales, biases, x, y, m, n, k, dtype);
}

int tfq_gemm_qg64(tfq_ctx* ctx, void* stream, const void* weights, const uint16_t* scales, const uint16_t* biases,
                  const uint16_t* x, uint16_t* y, uint32_t m, uint32_t n, uint32_t k, int dtype, uint32_t bits) {
    TFQ_REQUIRE_CTX(ctx);
    return ctx->qmm->encode(stream, weights, scales, biases, x, y, m, n, k, dtype, bits);
}

int tfq_gemm_qg64_path(tfq_ctx* ctx, void* stream, const void* weights, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* x, uint16_t* y, uint32_t m, uint32_t n,
                       uint32_t k, int dtype, uint32_t bits, int path) {
    TFQ_REQUIRE_CTX(ctx);
    return ctx->qmm->encode(stream, weights, scales, biases, x, y, m, n, k, dtype, bits, path);
}

int tfq_prefill_router(tfq_ctx* ctx, void* stream, const tfq_router* router, const uint16_t* hidden,
                       uint32_t hidden_stride, uint32_t T, uint32_t d, uint32_t top_k,
                       uint32_t* out_indices, uint16_t* out_weights, float* out_weights_f32,
                       float* logits_scratch) {
    TFQ_REQUIRE_CTX(ctx);
    if (!router) return fail(TFQ_E_INVAL, "null router");
    return ctx->prouter->encode_gemma4_block(stream, *router, hidden, hidden_stride, T, d, top_k,
                                             out_indices, out_weights, out_weights_f32,
                                             logits_scratch);
}

int tfq_moe_group(tfq_ctx* ctx, void* stream, const uint32_t* indices, const uint16_t* weights,
                  uint32_t T, uint32_t top_k, uint32_t num_experts, tfq_pair* sorted,
                  uint32_t* offsets, uint32_t* counts, tfq_tile* tiles, uint32_t* n_tiles,
                  uint32_t* status) {
    TFQ_REQUIRE_CTX(ctx);
    return ctx->grouping->encode(stream, indices, weights, T, top_k, num_experts, sorted, offsets,
                                 counts, tiles, n_tiles, status);
}

int tfq_moe_grouped(tfq_ctx* ctx, void* stream, const tfq_expert_pool* pool, const tfq_pair* sorted,
                    const tfq_tile* tiles, uint32_t* n_tiles, uint32_t max_tiles,
                    const uint16_t* hidden, uint32_t hidden_stride, uint32_t d, uint32_t f,
                    uint32_t top_k, uint16_t* act_scratch, uint16_t* route_partials) {
    TFQ_REQUIRE_CTX(ctx);
    if (!pool) return fail(TFQ_E_INVAL, "null pool");
    return ctx->grouped->encode(stream, *pool, sorted, tiles, n_tiles, max_tiles, hidden,
                                hidden_stride, d, f, top_k, act_scratch, route_partials);
}

int tfq_moe_combine(tfq_ctx* ctx, void* stream, const uint16_t* route_partials,
                    const uint16_t* route_weights, uint16_t* h2, uint32_t T, uint32_t top_k,
                    uint32_t d) {
    TFQ_REQUIRE_CTX(ctx);
    return ctx->grouped->encode_reduce_token_major(stream, route_partials, route_weights, h2, T,
                                                   top_k, d);
}

// Workspace of tfq_moe_prefill: 256-byte aligned segments in this order.
namespace {
struct PrefillLayout {
    size_t logits, sorted, tiles, offsets, counts, n_tiles, status, act, partials, total;
};
size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
PrefillLayout prefill_layout(uint32_t T, uint32_t k, uint32_t E, uint32_t d, uint32_t f) {
    PrefillLayout L{};
    const size_t n = (size_t)T * k;
    size_t cur = 0;
    auto take = [&](size_t bytes) { size_t at = cur; cur = align256(cur + bytes); return at; };
    L.logits = take((size_t)T * E * 4);
    L.sorted = take(n * 16);
    L.tiles = take((size_t)TFQ_MOE_MAX_TILES(T, k, E) * 16);
    L.offsets = take((size_t)E * 4);
    L.counts = take((size_t)E * 4);
    L.n_tiles = take(4 * TFQ_MOE_GROUP_STATE_WORDS);
    L.status = take(4);
    L.act = take(n * f * 2);
    L.partials = take(n * d * 2);
    L.total = cur;
    return L;
}
}  // namespace

size_t tfq_moe_prefill_workspace_bytes(uint32_t T, uint32_t top_k, uint32_t num_experts, uint32_t d,
                                       uint32_t f) {
    return prefill_layout(T, top_k, num_experts, d, f).total;
}

int tfq_moe_prefill(tfq_ctx* ctx, void* stream, const tfq_router* router, const tfq_expert_pool* pool,
                    const uint16_t* hidden, uint32_t hidden_stride, uint32_t T, uint32_t d, uint32_t f,
                    uint32_t top_k, uint16_t* h2, uint32_t* out_indices, uint16_t* out_weights,
                    void* workspace, size_t workspace_bytes) {
    TFQ_REQUIRE_CTX(ctx);
    if (!router || !pool || !workspace) return fail(TFQ_E_INVAL, "null router, pool or workspace");
    if (router->num_experts != pool->num_experts)
        return fail(TFQ_E_INVAL, "router has %u experts, pool %u", router->num_experts,
                    pool->num_experts);
    if (int rc = check_expert_pool(*pool, d, f)) return rc;     // before any launch: nothing queued on failure
    const uint32_t E = pool->num_experts;
    const PrefillLayout L = prefill_layout(T, top_k, E, d, f);
    if (workspace_bytes < L.total)
        return fail(TFQ_E_INVAL, "workspace of %zu bytes < %zu required", workspace_bytes, L.total);
    if (!aligned(workspace, 256)) return fail(TFQ_E_INVAL, "workspace must be 256-byte aligned");
    char* ws = static_cast<char*>(workspace);
    int rc = ctx->prouter->encode_gemma4_block(stream, *router, hidden, hidden_stride, T, d, top_k,
                                               out_indices, out_weights, nullptr,
                                               reinterpret_cast<float*>(ws + L.logits));
    if (rc) return rc;
    auto* sorted = reinterpret_cast<tfq_pair*>(ws + L.sorted);
    auto* tiles = reinterpret_cast<tfq_tile*>(ws + L.tiles);
    auto* n_tiles = reinterpret_cast<uint32_t*>(ws + L.n_tiles);
    rc = ctx->grouping->encode(stream, out_indices, out_weights, T, top_k, E, sorted,
                               reinterpret_cast<uint32_t*>(ws + L.offsets),
                               reinterpret_cast<uint32_t*>(ws + L.counts), tiles, n_tiles,
                               reinterpret_cast<uint32_t*>(ws + L.status));
    if (rc) return rc;
    auto* partials = reinterpret_cast<uint16_t*>(ws + L.partials);
    rc = ctx->grouped->encode(stream, *pool, sorted, tiles, n_tiles, TFQ_MOE_MAX_TILES(T, top_k, E),
                              hidden, hidden_stride, d, f, top_k,
                              reinterpret_cast<uint16_t*>(ws + L.act), partials);
    if (rc) return rc;
    return ctx->grouped->encode_reduce_token_major(stream, partials, out_weights, h2, T, top_k, d);
}

int tfq_group_pairs_host(const tfq_pair* pairs, int64_t n_pairs, int64_t query_count, int64_t top_k,
                         int64_t num_experts, int64_t tile_expert_count, const uint64_t* sort_keys,
                         int64_t n_sort_keys, tfq_pair* sorted, uint32_t* offsets, uint32_t* counts,
                         tfq_group* groups, int64_t* n_groups, tfq_group_tile* tiles,
                         int64_t* n_tiles, int64_t err[2]) {
    // PrefillMoEGrouping.swift:91-192: validation in the reference's order.
    err[0] = err[1] = 0;
    if (query_count < 0) { err[0] = query_count; return TFQ_GROUP_INVALID_QUERY_COUNT; }
    if (top_k <= 0) { err[0] = top_k; return TFQ_GROUP_INVALID_TOPK; }
    if (num_experts <= 0) { err[0] = num_experts; return TFQ_GROUP_INVALID_NUM_EXPERTS; }
    if (tile_expert_count < 1 || tile_expert_count > 16) {
        err[0] = tile_expert_count;
        return TFQ_GROUP_INVALID_TILE_EXPERT_COUNT;
    }
    if (sort_keys && n_sort_keys != num_experts) {
        err[0] = num_experts;
        err[1] = n_sort_keys;
        return TFQ_GROUP_SORT_KEY_COUNT_MISMATCH;
    }
    const int64_t expected = query_count * top_k;
    if (n_pairs != expected) {
        err[0] = expected;
        err[1] = n_pairs;
        return TFQ_GROUP_PAIR_COUNT_MISMATCH;
    }
    std::vector<uint8_t> seen((size_t)std::max<int64_t>(expected, 1), 0);
    for (int64_t i = 0; i < n_pairs; ++i) {
        const tfq_pair& p = pairs[i];
        if ((int64_t)p.token >= query_count) { err[0] = p.token; return TFQ_GROUP_TOKEN_OUT_OF_RANGE; }
        if ((int64_t)p.rank >= top_k) { err[0] = p.rank; return TFQ_GROUP_RANK_OUT_OF_RANGE; }
        if ((int64_t)p.expert >= num_experts) { err[0] = p.expert; return TFQ_GROUP_EXPERT_OUT_OF_RANGE; }
        const int64_t key = (int64_t)p.token * top_k + p.rank;
        if (seen[key]) {
            err[0] = p.token;
            err[1] = p.rank;
            return TFQ_GROUP_DUPLICATE_TOKEN_RANK;
        }
        seen[key] = 1;
    }
    std::copy(pairs, pairs + n_pairs, sorted);
    std::sort(sorted, sorted + n_pairs, [&](const tfq_pair& a, const tfq_pair& b) {
        if (sort_keys) {
            const uint64_t ka = sort_keys[a.expert], kb = sort_keys[b.expert];
            if (ka != kb) return ka < kb;
        }
        if (a.expert != b.expert) return a.expert < b.expert;
        if (a.token != b.token) return a.token < b.token;
        return a.rank < b.rank;
    });
    for (int64_t e = 0; e < num_experts; ++e) {
        offsets[e] = 0xFFFFFFFFu;
        counts[e] = 0;
    }
    int64_t ng = 0;
    for (int64_t i = 0; i < n_pairs;) {
        const uint32_t expert = sorted[i].expert;
        const int64_t start = i;
        while (i < n_pairs && sorted[i].expert == expert) ++i;
        offsets[expert] = (uint32_t)start;
        counts[expert] = (uint32_t)(i - start);
        groups[ng++] = {expert, (uint32_t)start, (uint32_t)(i - start)};
    }
    int64_t nt = 0;
    for (int64_t gs = 0; gs < ng;) {
        const int64_t ge = std::min(ng, gs + tile_expert_count);
        const uint32_t ps = groups[gs].pair_start;
        const uint32_t pe = groups[ge - 1].pair_start + groups[ge - 1].pair_count;
        tiles[nt++] = {(uint32_t)gs, (uint32_t)(ge - gs), ps, pe - ps};
        gs = ge;
    }
    *n_groups = ng;
    *n_tiles = nt;
    return TFQ_GROUP_OK;
}

int tfq_convert_bf16_to_f16(tfq_ctx* ctx, void* stream, const uint16_t* src, uint16_t* dst,
                            uint64_t count, uint32_t* inexact_count_dev) {
    TFQ_REQUIRE_CTX(ctx);
    if (count == 0) return TFQ_OK;
    if (!src || !dst) return fail(TFQ_E_INVAL, "null pointer argument");
    if (!aligned(src, 2) || !aligned(dst, 2)) return fail(TFQ_E_INVAL, "2-byte alignment required");
    uint64_t blocks = (count + 255) / 256;
    uint32_t grid = blocks > 2048 ? 2048u : (uint32_t)blocks;
    void* args[] = {&src, &dst, &count, &inexact_count_dev};
    return launch(ctx->module.get("tfq_convert_bf16_f16"), grid, 256, 0, stream, args,
                  "tfq_convert_bf16_f16");
}

int tfq_read_ceiling(tfq_ctx* ctx, void* stream, const void* src, uint64_t bytes, uint32_t* sink,
                     uint32_t sink_blocks) {
    TFQ_REQUIRE_CTX(ctx);
    if (!src || !sink || sink_blocks == 0) return fail(TFQ_E_INVAL, "null pointer or empty sink");
    if (!aligned(src, 16) || bytes % 16) return fail(TFQ_E_INVAL, "src and bytes must be 16-byte aligned");
    const uint64_t n16 = bytes / 16;
    // four 16-byte loads per lane in one pass while the sink allows it (one
    // load per lane, four times the blocks, measured slower: 6.5 against
    // 5.1 us for 4.47 MB cold), else more passes
    uint64_t blocks = (n16 + 256 * 4 - 1) / (256 * 4);
    if (blocks > sink_blocks) blocks = sink_blocks;
    if (blocks < 1) blocks = 1;
    uint32_t grid = (uint32_t)blocks;
    void* args[] = {&src, (void*)&n16, &sink};
    return launch(ctx->module.get("tfq_read_ceiling"), grid, 256, 0, stream, args,
                  "tfq_read_ceiling");
}

// ------------------------------------------------------------ runtime ----

int tfq_rt_device_count(int* count) { return hip_check(hipGetDeviceCount(count), "hipGetDeviceCount"); }
int tfq_rt_set_device(int device) { return hip_check(hipSetDevice(device), "hipSetDevice"); }

int tfq_rt_device_info(char* name, size_t name_len, char* arch, size_t arch_len) {
    int dev = 0;
    int rc = hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    hipDeviceProp_t prop;
    rc = hip_check(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
    if (rc) return rc;
    if (name && name_len) std::snprintf(name, name_len, "%s", prop.name);
    if (arch && arch_len) std::snprintf(arch, arch_len, "%s", prop.gcnArchName);
    return TFQ_OK;
}

int tfq_rt_malloc(void** ptr, size_t bytes) { return hip_check(hipMalloc(ptr, bytes), "hipMalloc"); }
int tfq_rt_free(void* ptr) { return hip_check(hipFree(ptr), "hipFree"); }
int tfq_rt_memcpy_htod(void* dst, const void* src, size_t bytes) {
    return hip_check(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpyHtoD");
}
int tfq_rt_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    return hip_check(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpyDtoH");
}
int tfq_rt_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream) {
    return hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream),
                     "hipMemcpyDtoD");
}
int tfq_rt_memset(void* dst, int value, size_t bytes) {
    // hipMemset of device memory may return before the fill is done, and the
    // null stream does not order work on the non-blocking streams these
    // bindings create: wait for it, as the header promises
    int rc = hip_check(hipMemset(dst, value, bytes), "hipMemset");
    if (rc) return rc;
    return hip_check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
}
int tfq_rt_stream_create(void** stream) {
    return hip_check(hipStreamCreateWithFlags((hipStream_t*)stream, hipStreamNonBlocking),
                     "hipStreamCreate");
}
int tfq_rt_stream_destroy(void* stream) {
    return hip_check(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
}
int tfq_rt_stream_sync(void* stream) {
    return hip_check(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}
int tfq_rt_device_sync(void) { return hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize"); }
int tfq_rt_event_create(void** event) {
    return hip_check(hipEventCreate((hipEvent_t*)event), "hipEventCreate");
}
int tfq_rt_event_destroy(void* event) {
    return hip_check(hipEventDestroy((hipEvent_t)event), "hipEventDestroy");
}
int tfq_rt_event_record(void* event, void* stream) {
    return hip_check(hipEventRecord((hipEvent_t)event, (hipStream_t)stream), "hipEventRecord");
}
int tfq_rt_event_sync(void* event) {
    return hip_check(hipEventSynchronize((hipEvent_t)event), "hipEventSynchronize");
}
int tfq_rt_event_elapsed_ms(float* ms, void* start, void* end) {
    return hip_check(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end),
                     "hipEventElapsedTime");
}
int tfq_rt_capture_begin(void* stream) {
    return hip_check(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal),
                     "hipStreamBeginCapture");
}
int tfq_rt_capture_end(void* stream, void** graph_exec) {
    hipGraph_t g = nullptr;
    int rc = hip_check(hipStreamEndCapture((hipStream_t)stream, &g), "hipStreamEndCapture");
    if (rc) return rc;
    hipGraphExec_t ex = nullptr;
    rc = hip_check(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void)hipGraphDestroy(g);
    if (rc) return rc;
    *graph_exec = ex;
    return TFQ_OK;
}
int tfq_rt_graph_launch(void* graph_exec, void* stream) {
    return hip_check(hipGraphLaunch((hipGraphExec_t)graph_exec, (hipStream_t)stream),
                     "hipGraphLaunch");
}
int tfq_rt_graph_destroy(void* graph_exec) {
    return hip_check(hipGraphExecDestroy((hipGraphExec_t)graph_exec), "hipGraphExecDestroy");
}

}  // extern "C"
