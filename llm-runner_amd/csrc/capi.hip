// capi.hip - the C-ABI boundary (include/llmr_hip.h): context, memory and the
// hot-path ops. Every entry point validates its arguments before anything is
// launched, so a bad call returns an error instead of reading out of bounds.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "llmr_hip.h"
#include "llmr_internal.h"

struct llmr_context {
    int device;
    int num_cus;
    hipStream_t own;
    hipStream_t cur;
    void* ws;         // library workspace (the SwiGLU's f32-input and fallback paths), grow-only
    size_t ws_bytes;
};

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_err[0] = '\0';
    return LLMR_OK;
}

#define LLMR_HIP_CHECK(expr)                                                                  \
    do {                                                                                      \
        hipError_t e_ = (expr);                                                               \
        if (e_ != hipSuccess) return fail(LLMR_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int check_ctx(llmr_context* ctx) {
    if (!ctx) return fail(LLMR_ERR_INVALID_ARG, "null context");
    LLMR_HIP_CHECK(hipSetDevice(ctx->device));
    return LLMR_OK;
}

bool is_act_type(uint32_t t) { return t == LLMR_GGML_F32 || t == LLMR_GGML_F16 || t == LLMR_GGML_BF16; }

// Weight-type and in_dim preconditions shared by dequant and GEMM
// (the reference assumes K % 32 for Q8_0 and K % 256 for Q4_K: llm.slang:1650,2284).
int check_weight(const void* w, uint32_t wtype, uint32_t in_dim) {
    if (!w) return fail(LLMR_ERR_INVALID_ARG, "null weight pointer");
    if (wtype != LLMR_GGML_Q8_0 && wtype != LLMR_GGML_Q4_K)
        return fail(LLMR_ERR_UNSUPPORTED, "weight type %u not implemented (Q8_0=8, Q4_K=12)", wtype);
    if (!aligned(w, 4)) return fail(LLMR_ERR_INVALID_ARG, "weight pointer must be 4-byte aligned");
    if (in_dim == 0) return fail(LLMR_ERR_INVALID_ARG, "in_dim must be > 0");
    if (wtype == LLMR_GGML_Q8_0 && in_dim % 32)
        return fail(LLMR_ERR_INVALID_ARG, "Q8_0 needs in_dim %% 32 == 0 (got %u)", in_dim);
    if (wtype == LLMR_GGML_Q4_K && in_dim % 256)
        return fail(LLMR_ERR_INVALID_ARG, "Q4_K needs in_dim %% 256 == 0 (got %u)", in_dim);
    return LLMR_OK;
}

}  // namespace

extern "C" {

const char* llmr_last_error(void) { return g_err; }

int llmr_create_context(int device_index, llmr_context** out_ctx) {
    if (!out_ctx) return fail(LLMR_ERR_INVALID_ARG, "null out_ctx");
    *out_ctx = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(LLMR_ERR_NO_DEVICE, "no HIP device");
    if (device_index < 0 || device_index >= n)
        return fail(LLMR_ERR_NO_DEVICE, "device index %d out of range [0, %d)", device_index, n);
    LLMR_HIP_CHECK(hipSetDevice(device_index));
    hipDeviceProp_t prop;
    LLMR_HIP_CHECK(hipGetDeviceProperties(&prop, device_index));
    llmr_context* c = new llmr_context;
    c->device = device_index;
    c->num_cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    hipError_t e = hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        return fail(LLMR_ERR_HIP, "hipStreamCreate: %s", hipGetErrorString(e));
    }
    c->cur = c->own;
    c->ws = nullptr;
    c->ws_bytes = 0;
    *out_ctx = c;
    return ok();
}

int llmr_destroy_context(llmr_context* ctx) {
    if (!ctx) return ok();
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->cur);
    (void)hipStreamSynchronize(ctx->own);
    (void)hipStreamDestroy(ctx->own);
    if (ctx->ws) (void)hipFree(ctx->ws);
    delete ctx;
    return ok();
}

int llmr_set_stream(llmr_context* ctx, void* hip_stream) {
    if (!ctx) return fail(LLMR_ERR_INVALID_ARG, "null context");
    ctx->cur = (hipStream_t)hip_stream;
    return ok();
}

void* llmr_get_stream(llmr_context* ctx) { return ctx ? (void*)ctx->cur : nullptr; }

int llmr_alloc(llmr_context* ctx, size_t bytes, void** out) {
    if (int r = check_ctx(ctx)) return r;
    if (!out) return fail(LLMR_ERR_INVALID_ARG, "null out pointer");
    *out = nullptr;
    if (bytes == 0) return ok();
    LLMR_HIP_CHECK(hipMalloc(out, bytes));
    return ok();
}

int llmr_free(llmr_context* ctx, void* p) {
    if (int r = check_ctx(ctx)) return r;
    if (!p) return ok();
    LLMR_HIP_CHECK(hipStreamSynchronize(ctx->cur));
    LLMR_HIP_CHECK(hipFree(p));
    return ok();
}

int llmr_upload(llmr_context* ctx, void* dst, const void* src, size_t bytes) {
    if (int r = check_ctx(ctx)) return r;
    if (bytes == 0) return ok();
    if (!dst || !src) return fail(LLMR_ERR_INVALID_ARG, "null pointer");
    LLMR_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->cur));
    LLMR_HIP_CHECK(hipStreamSynchronize(ctx->cur));
    return ok();
}

int llmr_download(llmr_context* ctx, void* dst, const void* src, size_t bytes) {
    if (int r = check_ctx(ctx)) return r;
    if (bytes == 0) return ok();
    if (!dst || !src) return fail(LLMR_ERR_INVALID_ARG, "null pointer");
    LLMR_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->cur));
    LLMR_HIP_CHECK(hipStreamSynchronize(ctx->cur));
    return ok();
}

int llmr_sync(llmr_context* ctx) {
    if (int r = check_ctx(ctx)) return r;
    LLMR_HIP_CHECK(hipStreamSynchronize(ctx->cur));
    return ok();
}

size_t llmr_ggml_row_bytes(uint32_t type, uint32_t n) {
    switch (type) {
        case LLMR_GGML_F32: return (size_t)n * 4;
        case LLMR_GGML_F16:
        case LLMR_GGML_BF16: return (size_t)n * 2;
        case LLMR_GGML_Q8_0: return n % 32 ? 0 : (size_t)(n / 32) * 34;
        case LLMR_GGML_Q4_K: return n % 256 ? 0 : (size_t)(n / 256) * 144;
        default: return 0;
    }
}

static int dequant_common(llmr_context* ctx, const void* w, uint32_t wtype, uint32_t n_rows,
                          uint32_t in_dim, uint32_t row_offset, void* out, bool operand) {
    if (int r = check_ctx(ctx)) return r;
    if (int r = check_weight(w, wtype, in_dim)) return r;
    if (!out) return fail(LLMR_ERR_INVALID_ARG, "null output pointer");
    if (!aligned(out, 16)) return fail(LLMR_ERR_INVALID_ARG, "output pointer must be 16-byte aligned");
    if ((uint64_t)row_offset + n_rows > 0xffffffffull)
        return fail(LLMR_ERR_INVALID_ARG, "row_offset + n_rows overflows");
    hipError_t e = operand
        ? llmr::launch_dequant_operand_f16(w, wtype, n_rows, in_dim, row_offset, (uint16_t*)out, ctx->cur)
        : llmr::launch_dequant_f32(w, wtype, n_rows, in_dim, row_offset, (float*)out, ctx->cur);
    if (e != hipSuccess) return fail(LLMR_ERR_HIP, "dequant launch: %s", hipGetErrorString(e));
    return ok();
}

int llmr_dequant(llmr_context* ctx, const void* w, uint32_t wtype, uint32_t n_rows, uint32_t in_dim,
                 uint32_t row_offset, float* out) {
    return dequant_common(ctx, w, wtype, n_rows, in_dim, row_offset, out, false);
}

int llmr_dequant_operand_f16(llmr_context* ctx, const void* w, uint32_t wtype, uint32_t n_rows,
                             uint32_t in_dim, uint32_t row_offset, uint16_t* out) {
    return dequant_common(ctx, w, wtype, n_rows, in_dim, row_offset, out, true);
}

int llmr_batch_matmul(llmr_context* ctx, const void* weight, uint32_t wtype, const void* input,
                      uint32_t xtype, float* output, uint32_t out_dim, uint32_t in_dim,
                      uint32_t seq_len, uint32_t row_offset) {
    if (int r = check_ctx(ctx)) return r;
    if (int r = check_weight(weight, wtype, in_dim)) return r;
    if (!is_act_type(xtype))
        return fail(LLMR_ERR_UNSUPPORTED, "input type %u not supported (F32=0, F16=1, BF16=30)", xtype);
    if (seq_len == 0 || out_dim == 0) return ok();
    if (!input || !output) return fail(LLMR_ERR_INVALID_ARG, "null input/output pointer");
    if (!aligned(input, 16) || !aligned(output, 16))
        return fail(LLMR_ERR_INVALID_ARG, "input/output pointers must be 16-byte aligned");
    if ((uint64_t)row_offset + out_dim > 0xffffffffull)
        return fail(LLMR_ERR_INVALID_ARG, "row_offset + out_dim overflows");
    hipError_t e = llmr::launch_batch_matmul(weight, wtype, input, xtype, output, out_dim, in_dim, seq_len,
                                             row_offset, ctx->num_cus, ctx->cur);
    if (e != hipSuccess) return fail(LLMR_ERR_HIP, "batch_matmul launch: %s", hipGetErrorString(e));
    return ok();
}

int llmr_batch_matmul_pc(llmr_context* ctx, const void* weight, uint32_t wtype, const void* input,
                         uint32_t xtype, float* output, const llmr_batch_matmul_params* pc) {
    if (!pc) return fail(LLMR_ERR_INVALID_ARG, "null push constants");
    return llmr_batch_matmul(ctx, weight, wtype, input, xtype, output, pc->out_dim, pc->in_dim,
                             pc->seq_len, pc->row_offset);
}

int llmr_batch_matmul_swiglu(llmr_context* ctx, const void* weight_gate, const void* weight_up,
                              uint32_t wtype, const void* input, uint32_t xtype, float* output,
                              uint32_t out_dim, uint32_t in_dim, uint32_t seq_len) {
    if (int r = check_ctx(ctx)) return r;
    if (wtype != LLMR_GGML_Q8_0)
        return fail(LLMR_ERR_UNSUPPORTED, "SwiGLU GEMM needs Q8_0 gate and up weights (llm.slang:1777), got type %u",
                    wtype);
    if (int r = check_weight(weight_gate, wtype, in_dim)) return r;
    if (int r = check_weight(weight_up, wtype, in_dim)) return r;
    if (!is_act_type(xtype))
        return fail(LLMR_ERR_UNSUPPORTED, "input type %u not supported (F32=0, F16=1, BF16=30)", xtype);
    if (seq_len == 0 || out_dim == 0) return ok();
    if (!input || !output) return fail(LLMR_ERR_INVALID_ARG, "null input/output pointer");
    if (!aligned(input, 16) || !aligned(output, 16))
        return fail(LLMR_ERR_INVALID_ARG, "input/output pointers must be 16-byte aligned");
    const size_t need = llmr::swiglu_workspace_bytes(wtype, xtype, out_dim, in_dim, seq_len);
    if (need > ctx->ws_bytes) {
        // hipFree waits for every launch that may still read the old workspace
        if (ctx->ws) LLMR_HIP_CHECK(hipFree(ctx->ws));
        ctx->ws = nullptr;
        ctx->ws_bytes = 0;
        LLMR_HIP_CHECK(hipMalloc(&ctx->ws, need));
        ctx->ws_bytes = need;
    }
    hipError_t e = llmr::launch_batch_matmul_swiglu(weight_gate, weight_up, wtype, input, xtype, output, out_dim,
                                                    in_dim, seq_len, ctx->num_cus, ctx->ws, ctx->cur);
    if (e != hipSuccess) return fail(LLMR_ERR_HIP, "batch_matmul_swiglu launch: %s", hipGetErrorString(e));
    return ok();
}

int llmr_batch_matmul_swiglu_pc(llmr_context* ctx, const void* weight_gate, const void* weight_up,
                                 uint32_t wtype, const void* input, uint32_t xtype, float* output,
                                 const llmr_batch_matmul_params* pc) {
    if (!pc) return fail(LLMR_ERR_INVALID_ARG, "null push constants");
    if (pc->row_offset != 0)
        return fail(LLMR_ERR_INVALID_ARG, "SwiGLU GEMM reads weight rows from 0 (row_offset must be 0, got %u)",
                    pc->row_offset);
    return llmr_batch_matmul_swiglu(ctx, weight_gate, weight_up, wtype, input, xtype, output, pc->out_dim,
                                    pc->in_dim, pc->seq_len);
}

int llmr_flash_attention(llmr_context* ctx, const void* q, const void* k, const void* v,
                         uint32_t xtype, float* out, uint32_t head_dim, uint32_t n_heads,
                         uint32_t seq_len, float scale) {
    if (int r = check_ctx(ctx)) return r;
    if (head_dim != 128)
        return fail(LLMR_ERR_INVALID_ARG, "head_dim must be 128 (flash_attn.slang:20), got %u", head_dim);
    if (!is_act_type(xtype))
        return fail(LLMR_ERR_UNSUPPORTED, "qkv type %u not supported (F32=0, F16=1, BF16=30)", xtype);
    if (!(scale > 0.0f) || !std::isfinite(scale))
        return fail(LLMR_ERR_INVALID_ARG, "scale must be positive and finite");
    if (seq_len == 0 || n_heads == 0) return ok();
    if (!q || !k || !v || !out) return fail(LLMR_ERR_INVALID_ARG, "null q/k/v/out pointer");
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16))
        return fail(LLMR_ERR_INVALID_ARG, "q/k/v/out pointers must be 16-byte aligned");
    if ((uint64_t)n_heads * ((seq_len + 127) / 128) > 0x7fffffffull)
        return fail(LLMR_ERR_INVALID_ARG, "grid too large");
    // one head's [S, 128] slab is addressed with 32-bit byte offsets
    if ((uint64_t)seq_len * 128u * (xtype == 0 ? 4u : 2u) > 0xffffffffull)
        return fail(LLMR_ERR_INVALID_ARG, "seq_len %u too large: one head must span < 4 GiB", seq_len);
    hipError_t e = llmr::launch_flash_attention(q, k, v, xtype, out, n_heads, seq_len, scale, ctx->cur);
    if (e != hipSuccess) return fail(LLMR_ERR_HIP, "flash_attention launch: %s", hipGetErrorString(e));
    return ok();
}

int llmr_flash_attention_pc(llmr_context* ctx, const void* q, const void* k, const void* v,
                            uint32_t xtype, float* out, const llmr_flash_attention_params* pc) {
    if (!pc) return fail(LLMR_ERR_INVALID_ARG, "null push constants");
    return llmr_flash_attention(ctx, q, k, v, xtype, out, pc->head_dim, pc->n_heads, pc->seq_len,
                                pc->scale);
}

}  // extern "C"
