// capi.hip - the C-ABI boundary (include/llmr_hip.h): context, memory and the
// hot-path ops. Every entry point validates its arguments before anything is
// launched, so a bad call returns an error instead of reading out of bounds.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "llmr_hip.h"
#include "llmr_internal.h"

struct llmr_context {
    int device;
    int num_cus;
    hipStream_t own;
    hipStream_t cur;
    // Library workspace, grow-only: f32 activations rounded to 16 bits, the
    // 16-bit weight images of the two-pass GEMM, split-K partials, the
    // fallback paths' f32 intermediates. A call on another stream than the
    // last user (ws_stream) waits for it through ws_done, recorded when the
    // context switched away from that stream.
    void* ws;
    size_t ws_bytes;
    hipEvent_t ws_done;
    hipStream_t ws_stream;
    bool ws_used;
    // The same ordering for the device's fixed no-allocation scratch, as far
    // as this context's calls go: a llmr_batch_matmul_noalloc call on another
    // stream than the last one waits for scr_done, recorded when the context
    // left that stream.
    hipEvent_t scr_done;
    hipStream_t scr_stream;
    bool scr_used;
};

// The no-allocation GEMM's scratch (llmr_batch_matmul_noalloc): a fixed
// device array each GPU holds from the library's load to the end of the
// process. Host code never uses the array's name as an address (on the host
// it is only a handle): the device address comes from hipGetSymbolAddress,
// once per device, at the first context creation on that device.
constexpr size_t kNoAllocScratchBytes = LLMR_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

thread_local char g_err[512] = "";

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on the current device `dev` (resolved once).
hipError_t resolve_scratch(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch[dev]) return hipSuccess;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess) g_scratch[dev] = p;
    return e;
}

void* scratch_ptr(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return g_scratch[dev];
}

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

int check_rows(const void* p, const char* what, uint32_t stride, uint32_t width) {
    if (!p) return fail(LLMR_ERR_INVALID_ARG, "null %s pointer", what);
    if (!aligned(p, 16)) return fail(LLMR_ERR_INVALID_ARG, "%s pointer must be 16-byte aligned", what);
    if (stride % 4) return fail(LLMR_ERR_INVALID_ARG, "%s row stride must be a multiple of 4 (got %u)", what, stride);
    if (stride < width) return fail(LLMR_ERR_INVALID_ARG, "%s row stride %u < row width %u", what, stride, width);
    return LLMR_OK;
}

int check_vec(const void* p, const char* what, bool required) {
    if (!p) return required ? fail(LLMR_ERR_INVALID_ARG, "null %s pointer", what) : LLMR_OK;
    if (!aligned(p, 16)) return fail(LLMR_ERR_INVALID_ARG, "%s pointer must be 16-byte aligned", what);
    return LLMR_OK;
}

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

namespace llmr {
// The error record for the host-only sources (gguf_file.cpp): sets
// llmr_last_error's message ("" on success) and returns code.
int set_error(int code, const char* msg) { return fail(code, "%s", msg); }
}  // namespace llmr

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
    LLMR_HIP_CHECK(resolve_scratch(device_index));
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
    c->ws_stream = nullptr;
    c->ws_used = false;
    c->scr_stream = nullptr;
    c->scr_used = false;
    e = hipEventCreateWithFlags(&c->ws_done, hipEventDisableTiming);
    if (e != hipSuccess) {
        (void)hipStreamDestroy(c->own);
        delete c;
        return fail(LLMR_ERR_HIP, "hipEventCreate: %s", hipGetErrorString(e));
    }
    e = hipEventCreateWithFlags(&c->scr_done, hipEventDisableTiming);
    if (e != hipSuccess) {
        (void)hipEventDestroy(c->ws_done);
        (void)hipStreamDestroy(c->own);
        delete c;
        return fail(LLMR_ERR_HIP, "hipEventCreate: %s", hipGetErrorString(e));
    }
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
    (void)hipEventDestroy(ctx->ws_done);
    (void)hipEventDestroy(ctx->scr_done);
    delete ctx;
    return ok();
}

int llmr_set_stream(llmr_context* ctx, void* hip_stream) {
    if (!ctx) return fail(LLMR_ERR_INVALID_ARG, "null context");
    const hipStream_t s = (hipStream_t)hip_stream;
    // leaving the stream that last used the workspace: mark the end of its
    // work for the next workspace user on another stream
    if (s != ctx->cur && ctx->ws_used && ctx->ws_stream == ctx->cur) {
        LLMR_HIP_CHECK(hipSetDevice(ctx->device));
        LLMR_HIP_CHECK(hipEventRecord(ctx->ws_done, ctx->cur));
    }
    // the same for the no-allocation scratch
    if (s != ctx->cur && ctx->scr_used && ctx->scr_stream == ctx->cur) {
        LLMR_HIP_CHECK(hipSetDevice(ctx->device));
        LLMR_HIP_CHECK(hipEventRecord(ctx->scr_done, ctx->cur));
    }
    ctx->cur = s;
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

// Makes the context workspace hold `need` bytes for a call about to be issued
// on the current stream. When the workspace was last used on another stream,
// the call first waits for ws_done, which llmr_set_stream recorded on that
// stream when the context left it (after everything issued there, the last
// use included); then the workspace grows if needed (hipFree waits for every
// launch that may still use the old one). Calls that stay on one stream
// record and wait for nothing.
static int acquire_workspace(llmr_context* ctx, size_t need) {
    if (need == 0) return LLMR_OK;
    if (ctx->ws_used && ctx->ws_stream != ctx->cur) LLMR_HIP_CHECK(hipStreamWaitEvent(ctx->cur, ctx->ws_done, 0));
    if (need > ctx->ws_bytes) {
        if (ctx->ws) LLMR_HIP_CHECK(hipFree(ctx->ws));
        ctx->ws = nullptr;
        ctx->ws_bytes = 0;
        LLMR_HIP_CHECK(hipMalloc(&ctx->ws, need));
        ctx->ws_bytes = need;
    }
    return LLMR_OK;
}

// Marks the workspace as used by the work just issued on the current stream.
static int release_workspace(llmr_context* ctx, size_t need) {
    if (need == 0) return LLMR_OK;
    ctx->ws_stream = ctx->cur;
    ctx->ws_used = true;
    return LLMR_OK;
}

// Argument checks of llmr_batch_matmul and its no-allocation variant.
static int check_batch_matmul(llmr_context* ctx, const void* weight, uint32_t wtype, const void* input,
                              uint32_t xtype, const float* output, uint32_t out_dim, uint32_t in_dim,
                              uint32_t seq_len, uint32_t row_offset) {
    if (int r = check_ctx(ctx)) return r;
    if (int r = check_weight(weight, wtype, in_dim)) return r;
    if (!is_act_type(xtype))
        return fail(LLMR_ERR_UNSUPPORTED, "input type %u not supported (F32=0, F16=1, BF16=30)", xtype);
    if (seq_len == 0 || out_dim == 0) return LLMR_OK;
    if (!input || !output) return fail(LLMR_ERR_INVALID_ARG, "null input/output pointer");
    if (!aligned(input, 16) || !aligned(output, 16))
        return fail(LLMR_ERR_INVALID_ARG, "input/output pointers must be 16-byte aligned");
    if ((uint64_t)row_offset + out_dim > 0xffffffffull)
        return fail(LLMR_ERR_INVALID_ARG, "row_offset + out_dim overflows");
    return LLMR_OK;
}

int llmr_batch_matmul(llmr_context* ctx, const void* weight, uint32_t wtype, const void* input,
                      uint32_t xtype, float* output, uint32_t out_dim, uint32_t in_dim,
                      uint32_t seq_len, uint32_t row_offset) {
    if (int r = check_batch_matmul(ctx, weight, wtype, input, xtype, output, out_dim, in_dim, seq_len, row_offset))
        return r;
    if (seq_len == 0 || out_dim == 0) return ok();
    const size_t need = llmr::batch_matmul_workspace_bytes(wtype, xtype, out_dim, in_dim, seq_len, ctx->num_cus);
    if (int r = acquire_workspace(ctx, need)) return r;
    hipError_t e = llmr::launch_batch_matmul(weight, wtype, input, xtype, output, out_dim, in_dim, seq_len,
                                             row_offset, ctx->num_cus, ctx->ws, ctx->cur);
    if (e != hipSuccess) return fail(LLMR_ERR_HIP, "batch_matmul launch: %s", hipGetErrorString(e));
    if (int r = release_workspace(ctx, need)) return r;
    return ok();
}

int llmr_batch_matmul_pc(llmr_context* ctx, const void* weight, uint32_t wtype, const void* input,
                         uint32_t xtype, float* output, const llmr_batch_matmul_params* pc) {
    if (!pc) return fail(LLMR_ERR_INVALID_ARG, "null push constants");
    return llmr_batch_matmul(ctx, weight, wtype, input, xtype, output, pc->out_dim, pc->in_dim,
                             pc->seq_len, pc->row_offset);
}

int llmr_batch_matmul_noalloc(llmr_context* ctx, const void* weight, uint32_t wtype, const void* input,
                              uint32_t xtype, float* output, uint32_t out_dim, uint32_t in_dim, uint32_t seq_len,
                              uint32_t row_offset) {
    if (int r = check_batch_matmul(ctx, weight, wtype, input, xtype, output, out_dim, in_dim, seq_len, row_offset))
        return r;
    if (seq_len == 0 || out_dim == 0) return ok();
    // the plan keeps within the scratch: smaller forms (one-pass kernels
    // instead of a weight image, fewer K splits, the tiled kernel reading f32
    // activations in place) where the usual plan needs more
    const size_t need = llmr::batch_matmul_workspace_bytes(wtype, xtype, out_dim, in_dim, seq_len, ctx->num_cus,
                                                           kNoAllocScratchBytes);
    if (need > kNoAllocScratchBytes)
        return fail(LLMR_ERR_INVALID_ARG, "this GEMM needs %zu bytes of scratch, beyond the %zu the no-allocation "
                    "entry point holds; call llmr_batch_matmul", need, kNoAllocScratchBytes);
    void* const ptr = scratch_ptr(ctx->device);
    if (need > 0 && !ptr) return fail(LLMR_ERR_HIP, "scratch of device %d not resolved", ctx->device);
    if (need > 0 && ctx->scr_used && ctx->scr_stream != ctx->cur)
        LLMR_HIP_CHECK(hipStreamWaitEvent(ctx->cur, ctx->scr_done, 0));
    hipError_t e = llmr::launch_batch_matmul(weight, wtype, input, xtype, output, out_dim, in_dim, seq_len, row_offset,
                                             ctx->num_cus, ptr, ctx->cur, kNoAllocScratchBytes);
    if (e != hipSuccess) return fail(LLMR_ERR_HIP, "batch_matmul launch: %s", hipGetErrorString(e));
    if (need > 0) {
        ctx->scr_stream = ctx->cur;
        ctx->scr_used = true;
    }
    return ok();
}

int llmr_lora_correction(llmr_context* ctx, const llmr_lora* lora, float* scratch, const void* input,
                         uint32_t xtype, float* output, uint32_t in_dim, uint32_t out_dim, uint32_t seq_len,
                         uint32_t b_rows, uint32_t row_offset, uint32_t weight_row_offset) {
    if (int r = check_ctx(ctx)) return r;
    // dit.c3:1333-1334: no adapter, or a rank beyond the scratch the
    // reference sizes, leaves the base output as it is
    if (!lora || lora->rank == 0 || lora->rank > llmr::kMaxLoraRank) return ok();
    if (!is_act_type(xtype))
        return fail(LLMR_ERR_UNSUPPORTED, "input type %u not supported (F32=0, F16=1, BF16=30)", xtype);
    if (seq_len == 0) return ok();
    if (!lora->a || !lora->b || !scratch || !input || !output)
        return fail(LLMR_ERR_INVALID_ARG, "null LoRA, scratch, input or output pointer");
    if (in_dim == 0) return fail(LLMR_ERR_INVALID_ARG, "in_dim must be positive");
    if (b_rows == 0) b_rows = out_dim;
    if ((uint64_t)row_offset + b_rows > out_dim)
        return fail(LLMR_ERR_INVALID_ARG, "row_offset + b_rows (%u + %u) exceeds out_dim %u", row_offset, b_rows,
                    out_dim);
    hipError_t e = llmr::launch_lora_correction(lora->a, lora->b, lora->rank, lora->scale, scratch, input, xtype,
                                                output, in_dim, out_dim, seq_len, b_rows, row_offset,
                                                weight_row_offset, ctx->cur);
    if (e != hipSuccess) return fail(LLMR_ERR_HIP, "lora_correction launch: %s", hipGetErrorString(e));
    return ok();
}

int llmr_batch_matmul_lora(llmr_context* ctx, const void* weight, uint32_t wtype, const void* input, uint32_t xtype,
                           float* output, uint32_t out_dim, uint32_t in_dim, uint32_t seq_len, uint32_t row_offset,
                           const llmr_lora* lora, float* lora_scratch, uint32_t lora_b_rows,
                           uint32_t lora_row_offset, uint32_t lora_weight_row_offset) {
    // a GEMM on the two-pass kernel merges the LoRA (rank <= 64) into its
    // weight image; the rest runs the GEMM, then the exact correction
    if (int r = check_batch_matmul(ctx, weight, wtype, input, xtype, output, out_dim, in_dim, seq_len, row_offset))
        return r;
    const bool present = lora && lora->rank > 0 && lora->rank <= llmr::kMaxLoraRank && seq_len > 0 && out_dim > 0;
    const size_t need = present ? llmr::batch_matmul_lora_workspace_bytes(wtype, xtype, out_dim, in_dim, seq_len,
                                                                          lora->rank, ctx->num_cus)
                                : 0u;
    if (need == 0) {
        if (int r = llmr_batch_matmul(ctx, weight, wtype, input, xtype, output, out_dim, in_dim, seq_len, row_offset))
            return r;
        return llmr_lora_correction(ctx, lora, lora_scratch, input, xtype, output, in_dim, out_dim, seq_len,
                                    lora_b_rows, lora_row_offset, lora_weight_row_offset);
    }
    if (!lora->a || !lora->b) return fail(LLMR_ERR_INVALID_ARG, "null LoRA a or b pointer");
    const uint32_t b_rows = lora_b_rows ? lora_b_rows : out_dim;
    if ((uint64_t)lora_row_offset + b_rows > out_dim)
        return fail(LLMR_ERR_INVALID_ARG, "row_offset + b_rows (%u + %u) exceeds out_dim %u", lora_row_offset,
                    b_rows, out_dim);
    const llmr::LoraGemm l{lora->a, lora->b, lora->rank, lora->scale, b_rows, lora_row_offset,
                           lora_weight_row_offset};
    if (int r = acquire_workspace(ctx, need)) return r;
    hipError_t e = llmr::launch_batch_matmul_lora(weight, wtype, input, xtype, output, out_dim, in_dim, seq_len,
                                                  row_offset, l, ctx->num_cus, ctx->ws, ctx->cur);
    if (e != hipSuccess) return fail(LLMR_ERR_HIP, "batch_matmul_lora launch: %s", hipGetErrorString(e));
    if (int r = release_workspace(ctx, need)) return r;
    return ok();
}

int llmr_q8_lora_merge(llmr_context* ctx, void* weight, const float* a, const float* b, uint32_t in_dim,
                       uint32_t b_rows, uint32_t dst_row_offset, uint32_t rank, float scale) {
    if (int r = check_ctx(ctx)) return r;
    // lora_merge.c3:55-62: the merge takes in_dim % 256 == 0 and rank <= 256
    if (in_dim == 0 || in_dim % 256 != 0)
        return fail(LLMR_ERR_UNSUPPORTED, "LoRA merge needs in_dim %% 256 == 0 (got %u)", in_dim);
    if (rank == 0 || rank > llmr::kMaxLoraRank)
        return fail(LLMR_ERR_UNSUPPORTED, "LoRA merge needs 1 <= rank <= %u (got %u)", llmr::kMaxLoraRank, rank);
    if (b_rows == 0) return ok();
    if (!weight || !a || !b) return fail(LLMR_ERR_INVALID_ARG, "null weight, a or b pointer");
    if ((uint64_t)dst_row_offset + b_rows > 0xffffffffull)
        return fail(LLMR_ERR_INVALID_ARG, "dst_row_offset + b_rows overflows");
    hipError_t e = llmr::launch_q8_lora_merge(weight, a, b, in_dim, b_rows, dst_row_offset, rank, scale, ctx->cur);
    if (e != hipSuccess) return fail(LLMR_ERR_HIP, "q8_lora_merge launch: %s", hipGetErrorString(e));
    return ok();
}

// The head routing of llmr_batch_matmul_multi_qkv: checks `heads` against
// the call and turns a STORE epilogue into SPLIT_GELU with split = out_dim
// (no gelu columns), the form the kernels take.
static int check_qkv_heads(const llmr_qkv_heads_out* h, uint32_t out_dim, const llmr_matmul_job* jobs,
                           uint32_t n_jobs, llmr_matmul_epilogue& e) {
    if (h->n_heads == 0 || h->n_heads > 1024) return fail(LLMR_ERR_INVALID_ARG, "heads: n_heads must be in [1, 1024]");
    const uint32_t qkv = 3u * h->n_heads * 128u;
    if (e.kind == LLMR_EPI_GATED_RESIDUAL)
        return fail(LLMR_ERR_INVALID_ARG, "heads: not with a GATED_RESIDUAL epilogue");
    if (e.kind == LLMR_EPI_STORE) {
        if (out_dim != qkv)
            return fail(LLMR_ERR_INVALID_ARG, "heads: a STORE epilogue needs out_dim = 3 * n_heads * 128 = %u "
                        "(got %u)", qkv, out_dim);
        e = llmr_matmul_epilogue{LLMR_EPI_SPLIT_GELU, 0, out_dim, 0, LLMR_GGML_BF16};
    } else if (e.split != qkv) {
        return fail(LLMR_ERR_INVALID_ARG, "heads: split must be 3 * n_heads * 128 = %u (got %u)", qkv, e.split);
    }
    if (h->out_type != LLMR_GGML_F16 && h->out_type != LLMR_GGML_BF16)
        return fail(LLMR_ERR_UNSUPPORTED, "heads: out_type must be F16 or BF16 (got %u)", h->out_type);
    if (!(h->eps >= 0.0f) || !std::isfinite(h->eps))
        return fail(LLMR_ERR_INVALID_ARG, "heads: eps must be finite and >= 0");
    if (int r = check_vec(h->q, "heads q", true)) return r;
    if (int r = check_vec(h->k, "heads k", true)) return r;
    if (int r = check_vec(h->v, "heads v", true)) return r;
    if ((h->rope_cos == nullptr) != (h->rope_sin == nullptr))
        return fail(LLMR_ERR_INVALID_ARG, "heads: rope_cos and rope_sin must both be given or both be null");
    if (int r = check_vec(h->rope_cos, "heads rope_cos", false)) return r;
    if (int r = check_vec(h->rope_sin, "heads rope_sin", false)) return r;
    if ((uint64_t)h->seq_len * 256u > 0xffffffffull) return fail(LLMR_ERR_INVALID_ARG, "heads: seq_len too large");
    for (uint32_t i = 0; i < n_jobs; i++) {
        const llmr_qkv_heads_job hj = h->jobs ? h->jobs[i] : llmr_qkv_heads_job{nullptr, nullptr, 0};
        if (int r = check_vec(hj.q_norm, "heads q_norm", false)) return r;
        if (int r = check_vec(hj.k_norm, "heads k_norm", false)) return r;
        if ((uint64_t)hj.row0 + jobs[i].seq_len > h->seq_len)
            return fail(LLMR_ERR_INVALID_ARG, "heads: job %u: row0 + seq_len (%llu) > seq_len %u", i,
                        (unsigned long long)hj.row0 + jobs[i].seq_len, h->seq_len);
    }
    return LLMR_OK;
}

static int batch_matmul_multi_impl(llmr_context* ctx, uint32_t wtype, uint32_t xtype, uint32_t out_dim,
                                   uint32_t in_dim, const llmr_matmul_job* jobs, uint32_t n_jobs,
                                   const llmr_matmul_epilogue* epilogue, const void* const* images,
                                   const llmr_next_weight_images* next, const llmr_qkv_heads_out* heads = nullptr) {
    if (int r = check_ctx(ctx)) return r;
    llmr::NextImageSet nx{};
    if (next) {
        if (xtype != LLMR_GGML_F16 && xtype != LLMR_GGML_BF16)
            return fail(LLMR_ERR_INVALID_ARG, "next weight images need F16 or BF16 input");
        if (next->count == 0 || next->count > llmr::kMaxNextImages)
            return fail(LLMR_ERR_INVALID_ARG, "next: count must be 1 to %u", llmr::kMaxNextImages);
        for (uint32_t i = 0; i < next->count; i++) {
            const llmr_next_weight_image& m = next->image[i];
            if (m.in_dim % 64 || m.out_dim == 0)
                return fail(LLMR_ERR_INVALID_ARG, "next image %u: in_dim %% 64 == 0 and out_dim > 0 needed", i);
            if (m.swiglu > 1) return fail(LLMR_ERR_INVALID_ARG, "next image %u: swiglu must be 0 or 1", i);
            if (m.up_offset && !m.swiglu)
                return fail(LLMR_ERR_INVALID_ARG, "next image %u: up_offset needs swiglu 1", i);
            if (m.swiglu && m.up_offset && m.up_offset < m.out_dim)
                return fail(LLMR_ERR_INVALID_ARG, "next image %u: up_offset below out_dim (the up rows overlap the gate "
                            "rows)", i);
            const size_t need = llmr::w16_image_bytes(m.out_dim, m.in_dim, m.swiglu != 0);
            if (m.image_bytes < need)
                return fail(LLMR_ERR_INVALID_ARG, "next image %u holds %zu bytes, needs %zu", i, m.image_bytes,
                            need);
            if (int r = check_weight(m.weight, next->weight_type, m.in_dim)) return r;
            const uint64_t up = m.swiglu ? (m.up_offset ? m.up_offset : m.out_dim) : 0u;
            if ((uint64_t)m.row_offset + up + m.out_dim > 0xffffffffull)
                return fail(LLMR_ERR_INVALID_ARG, "next image %u: its last row overflows 32 bits", i);
            if (!m.image || !aligned(m.image, 256))
                return fail(LLMR_ERR_INVALID_ARG, "next image %u must be non-null and 256-byte aligned", i);
            for (uint32_t j = 0; j < i; j++)
                if (next->image[j].image == m.image)
                    return fail(LLMR_ERR_INVALID_ARG, "next images %u and %u are the same buffer", j, i);
            if (images)
                for (uint32_t j = 0; j < n_jobs; j++)
                    if (images[j] == m.image)
                        return fail(LLMR_ERR_INVALID_ARG, "next: image %u is also an image of this call", i);
            nx.w[i] = m.weight;
            nx.img[i] = m.image;
            nx.row_offset[i] = m.row_offset;
            nx.N[i] = m.out_dim;
            nx.K[i] = m.in_dim;
            nx.sw[i] = m.swiglu;
            nx.up[i] = m.up_offset;
        }
        nx.count = next->count;
        nx.wtype = next->weight_type;
    }
    if (!is_act_type(xtype))
        return fail(LLMR_ERR_UNSUPPORTED, "input type %u not supported (F32=0, F16=1, BF16=30)", xtype);
    if (n_jobs == 0 || out_dim == 0) {  // no GEMM: the next group's images alone
        if (!next) return ok();
        const hipError_t e = llmr::finish_next_images(nx, xtype, 0u, ctx->cur);
        return e == hipSuccess ? ok() : fail(LLMR_ERR_HIP, "weight image launch: %s", hipGetErrorString(e));
    }
    if (!jobs) return fail(LLMR_ERR_INVALID_ARG, "null jobs");
    if (n_jobs > 64) return fail(LLMR_ERR_INVALID_ARG, "at most 64 jobs per call (got %u)", n_jobs);
    llmr_matmul_epilogue e = epilogue ? *epilogue : llmr_matmul_epilogue{LLMR_EPI_STORE, 0, 0, 0, 0};
    if (e.kind > LLMR_EPI_SPLIT_SWIGLU) return fail(LLMR_ERR_INVALID_ARG, "unknown epilogue kind %u", e.kind);
    if (heads)
        if (int r = check_qkv_heads(heads, out_dim, jobs, n_jobs, e)) return r;
    const bool swiglu = e.kind == LLMR_EPI_SPLIT_SWIGLU;
    const bool split = e.kind == LLMR_EPI_SPLIT_GELU || swiglu;
    if (!split) e.split = out_dim;
    if (split && (e.split > out_dim || e.split % 8))
        return fail(LLMR_ERR_INVALID_ARG, "split must be a multiple of 8 and <= out_dim (got %u)", e.split);
    // SPLIT_SWIGLU: out_dim = split + 2 f, whole 256-row panels below split
    const uint32_t f2 = out_dim - e.split, n2 = swiglu ? f2 / 2u : f2;  // output2 columns
    if (swiglu && (e.split % 256 || f2 % 16 || f2 == 0))
        return fail(LLMR_ERR_INVALID_ARG, "SPLIT_SWIGLU needs split %% 256 == 0 and out_dim - split = 2 f, "
                    "f %% 8 == 0, f > 0 (got split %u, out_dim %u)", e.split, out_dim);
    if (e.ldy == 0) e.ldy = split ? e.split : out_dim;
    if (e.ldy2 == 0) e.ldy2 = n2;
    const uint32_t width = split ? e.split : out_dim;
    const bool plain = e.kind == LLMR_EPI_STORE && e.ldy == out_dim;
    if (!plain && out_dim % 4) return fail(LLMR_ERR_INVALID_ARG, "this epilogue needs out_dim %% 4 == 0");
    if (!plain && (e.ldy % 4 || e.ldy < width))
        return fail(LLMR_ERR_INVALID_ARG, "ldy must be a multiple of 4 and >= %u (got %u)", width, e.ldy);
    if (e.kind == LLMR_EPI_GATED_RESIDUAL && out_dim > llmr::kRowNormMaxDim)
        return fail(LLMR_ERR_INVALID_ARG, "GATED_RESIDUAL needs out_dim <= %u", llmr::kRowNormMaxDim);
    const bool has2 = split && e.split < out_dim;
    if (has2 && (e.ldy2 % 4 || e.ldy2 < n2))
        return fail(LLMR_ERR_INVALID_ARG, "ldy2 must be a multiple of 4 and >= %u", n2);
    if (has2 && e.output2_type != LLMR_GGML_BF16 && e.output2_type != LLMR_GGML_F16)
        return fail(LLMR_ERR_UNSUPPORTED, "output2_type must be BF16 or F16 (got %u)", e.output2_type);
    if ((uint64_t)e.ldy > 0xffffffffull / 4) return fail(LLMR_ERR_INVALID_ARG, "ldy too large");
    llmr::GemmJob gj[64];
    for (uint32_t i = 0; i < n_jobs; i++) {
        const llmr_matmul_job& j = jobs[i];
        if (int r = check_weight(j.weight, wtype, in_dim)) return r;
        if (j.seq_len && (!j.input || (!j.output && !heads && !(swiglu && e.split == 0))))
            return fail(LLMR_ERR_INVALID_ARG, "job %u: null input/output pointer", i);
        if (!aligned(j.input, 16) || !aligned(j.output, 16))
            return fail(LLMR_ERR_INVALID_ARG, "job %u: input/output pointers must be 16-byte aligned", i);
        if ((uint64_t)j.row_offset + out_dim > 0xffffffffull)
            return fail(LLMR_ERR_INVALID_ARG, "job %u: row_offset + out_dim overflows", i);
        if (e.kind == LLMR_EPI_GATED_RESIDUAL && j.gate && !aligned(j.gate, 16))
            return fail(LLMR_ERR_INVALID_ARG, "job %u: gate must be 16-byte aligned", i);
        if (has2 && j.seq_len && (!j.output2 || !aligned(j.output2, 16)))
            return fail(LLMR_ERR_INVALID_ARG, "job %u: output2 must be non-null and 16-byte aligned", i);
        if (images && (!images[i] || !aligned(images[i], 256)))
            return fail(LLMR_ERR_INVALID_ARG, "job %u: weight image must be non-null and 256-byte aligned", i);
        gj[i] = llmr::GemmJob{j.weight, j.input, j.output, e.kind == LLMR_EPI_GATED_RESIDUAL ? j.gate : nullptr,
                              has2 ? j.output2 : nullptr, j.seq_len, j.row_offset};
        if (heads && heads->jobs) {
            gj[i].q_norm = heads->jobs[i].q_norm;
            gj[i].k_norm = heads->jobs[i].k_norm;
            gj[i].row0 = heads->jobs[i].row0;
        }
    }
    if (images && (xtype == LLMR_GGML_F32 || in_dim % 64))
        return fail(LLMR_ERR_INVALID_ARG, "weight images need F16/BF16 input and in_dim %% 64 == 0");
    llmr::GemmHeads gh{};
    if (heads)
        gh = llmr::GemmHeads{heads->q,       heads->k,        heads->v,        heads->rope_cos, heads->rope_sin,
                             heads->n_heads, heads->seq_len, heads->out_type, heads->eps};
    const llmr::GemmEpilogue ge{e.kind, e.ldy, e.ldy2, e.split, has2 ? e.output2_type : (uint32_t)LLMR_GGML_BF16,
                                heads ? &gh : nullptr};
    const size_t need = llmr::batch_matmul_multi_workspace_bytes(wtype, xtype, out_dim, in_dim, gj, n_jobs, ge,
                                                                 ctx->num_cus, images != nullptr);
    if (int r = acquire_workspace(ctx, need)) return r;
    hipError_t err = llmr::launch_batch_matmul_multi(wtype, xtype, out_dim, in_dim, gj, n_jobs, ge, ctx->num_cus,
                                                     ctx->ws, ctx->cur, images, next ? &nx : nullptr);
    if (err != hipSuccess) return fail(LLMR_ERR_HIP, "batch_matmul_multi launch: %s", hipGetErrorString(err));
    if (int r = release_workspace(ctx, need)) return r;
    return ok();
}

int llmr_batch_matmul_multi(llmr_context* ctx, uint32_t wtype, uint32_t xtype, uint32_t out_dim, uint32_t in_dim,
                            const llmr_matmul_job* jobs, uint32_t n_jobs, const llmr_matmul_epilogue* epilogue) {
    return batch_matmul_multi_impl(ctx, wtype, xtype, out_dim, in_dim, jobs, n_jobs, epilogue, nullptr, nullptr);
}

int llmr_batch_matmul_multi_images(llmr_context* ctx, uint32_t wtype, uint32_t xtype, uint32_t out_dim,
                                   uint32_t in_dim, const llmr_matmul_job* jobs, uint32_t n_jobs,
                                   const llmr_matmul_epilogue* epilogue, const void* const* images,
                                   const llmr_next_weight_images* next) {
    return batch_matmul_multi_impl(ctx, wtype, xtype, out_dim, in_dim, jobs, n_jobs, epilogue, images, next);
}

int llmr_batch_matmul_multi_qkv(llmr_context* ctx, uint32_t wtype, uint32_t xtype, uint32_t out_dim,
                                uint32_t in_dim, const llmr_matmul_job* jobs, uint32_t n_jobs,
                                const llmr_matmul_epilogue* epilogue, const llmr_qkv_heads_out* heads,
                                const void* const* images, const llmr_next_weight_images* next) {
    if (!heads) return fail(LLMR_ERR_INVALID_ARG, "null heads");
    return batch_matmul_multi_impl(ctx, wtype, xtype, out_dim, in_dim, jobs, n_jobs, epilogue, images, next, heads);
}

size_t llmr_weight_image_bytes(uint32_t out_dim, uint32_t in_dim) {
    return in_dim % 64 ? 0u : llmr::w16_image_bytes(out_dim, in_dim, false);
}

size_t llmr_swiglu_weight_image_bytes(uint32_t n_out, uint32_t in_dim) {
    return in_dim % 64 ? 0u : llmr::w16_image_bytes(n_out, in_dim, true);
}

int llmr_build_weight_image(llmr_context* ctx, const void* weight, uint32_t wtype, uint32_t xtype, uint32_t out_dim,
                            uint32_t in_dim, uint32_t row_offset, void* image, size_t image_bytes) {
    if (int r = check_ctx(ctx)) return r;
    if (xtype != LLMR_GGML_F16 && xtype != LLMR_GGML_BF16)
        return fail(LLMR_ERR_UNSUPPORTED, "weight images are built for F16 or BF16 input (got %u)", xtype);
    if (in_dim % 64) return fail(LLMR_ERR_INVALID_ARG, "in_dim must be a multiple of 64 (got %u)", in_dim);
    if (out_dim == 0) return ok();
    if (int r = check_weight(weight, wtype, in_dim)) return r;
    if ((uint64_t)row_offset + out_dim > 0xffffffffull)
        return fail(LLMR_ERR_INVALID_ARG, "row_offset + out_dim overflows");
    if (!image || !aligned(image, 256)) return fail(LLMR_ERR_INVALID_ARG, "image must be non-null, 256-byte aligned");
    const size_t need = llmr::w16_image_bytes(out_dim, in_dim, false);
    if (image_bytes < need)
        return fail(LLMR_ERR_INVALID_ARG, "image holds %zu bytes, needs %zu", image_bytes, need);
    const hipError_t err = llmr::launch_w16_image(weight, nullptr, wtype, xtype, image, out_dim, in_dim, row_offset,
                                                  ctx->cur);
    if (err != hipSuccess) return fail(LLMR_ERR_HIP, "weight image launch: %s", hipGetErrorString(err));
    return ok();
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
    const size_t need = llmr::swiglu_workspace_bytes(wtype, xtype, out_dim, in_dim, seq_len, ctx->num_cus);
    if (int r = acquire_workspace(ctx, need)) return r;
    hipError_t e = llmr::launch_batch_matmul_swiglu(weight_gate, weight_up, wtype, input, xtype, output, out_dim,
                                                    in_dim, seq_len, ctx->num_cus, ctx->ws, ctx->cur);
    if (e != hipSuccess) return fail(LLMR_ERR_HIP, "batch_matmul_swiglu launch: %s", hipGetErrorString(e));
    if (int r = release_workspace(ctx, need)) return r;
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

static int flash_attention_impl(llmr_context* ctx, const void* q, const void* k, const void* v, uint32_t xtype,
                                void* out, uint32_t out_type, uint32_t out_stride, uint32_t head_dim,
                                uint32_t n_heads, uint32_t seq_len, float scale) {
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
    if ((uint64_t)seq_len * 128u * (xtype == LLMR_GGML_F32 ? 4u : 2u) > 0xffffffffull)
        return fail(LLMR_ERR_INVALID_ARG, "seq_len %u too large: one head must span < 4 GiB", seq_len);
    if (!is_act_type(out_type))
        return fail(LLMR_ERR_UNSUPPORTED, "output type %u not supported (F32=0, F16=1, BF16=30)", out_type);
    if (out_stride % 8u || (uint64_t)out_stride < (uint64_t)n_heads * head_dim)
        return fail(LLMR_ERR_INVALID_ARG, "out_stride must be a multiple of 8 and >= n_heads * head_dim (got %u)",
                    out_stride);
    const size_t need = llmr::flash_attention_workspace_bytes(xtype, n_heads, seq_len);
    if (int r = acquire_workspace(ctx, need)) return r;
    hipError_t e = llmr::launch_flash_attention(q, k, v, xtype, out, out_type, out_stride, n_heads, seq_len, scale,
                                                ctx->ws, ctx->cur);
    if (e != hipSuccess) return fail(LLMR_ERR_HIP, "flash_attention launch: %s", hipGetErrorString(e));
    if (int r = release_workspace(ctx, need)) return r;
    return ok();
}

int llmr_flash_attention(llmr_context* ctx, const void* q, const void* k, const void* v,
                         uint32_t xtype, float* out, uint32_t head_dim, uint32_t n_heads,
                         uint32_t seq_len, float scale) {
    return flash_attention_impl(ctx, q, k, v, xtype, out, LLMR_GGML_F32, n_heads * head_dim, head_dim, n_heads,
                                seq_len, scale);
}

int llmr_flash_attention_rows(llmr_context* ctx, const void* q, const void* k, const void* v, uint32_t xtype,
                              void* out, uint32_t out_type, uint32_t out_stride, uint32_t head_dim,
                              uint32_t n_heads, uint32_t seq_len, float scale) {
    return flash_attention_impl(ctx, q, k, v, xtype, out, out_type, out_stride, head_dim, n_heads, seq_len, scale);
}

int llmr_flash_attention_pc(llmr_context* ctx, const void* q, const void* k, const void* v,
                            uint32_t xtype, float* out, const llmr_flash_attention_params* pc) {
    if (!pc) return fail(LLMR_ERR_INVALID_ARG, "null push constants");
    return llmr_flash_attention(ctx, q, k, v, xtype, out, pc->head_dim, pc->n_heads, pc->seq_len,
                                pc->scale);
}

}  // extern "C"

// --- block glue ---------------------------------------------------------------

namespace {

// A row-major [rows, stride] operand accessed in 4-element vectors over `width` columns.
int check_dim(uint32_t dim) {
    if (dim == 0 || dim % 4 || dim > llmr::kRowNormMaxDim)
        return fail(LLMR_ERR_INVALID_ARG, "dim must be a positive multiple of 4 and <= %u (got %u)",
                    llmr::kRowNormMaxDim, dim);
    return LLMR_OK;
}

int launched(hipError_t e, const char* op) {
    if (e != hipSuccess) return fail(LLMR_ERR_HIP, "%s launch: %s", op, hipGetErrorString(e));
    return ok();
}

int row_norm_common(llmr_context* ctx, bool ln, const float* x, uint32_t x_stride, const float* weight,
                    const float* mod_scale, const float* mod_shift, void* out, uint32_t out_type,
                    uint32_t out_stride, uint32_t dim, uint32_t n_rows, float eps, uint32_t split = ~0u,
                    const float* mod_scale2 = nullptr, const float* mod_shift2 = nullptr) {
    if (int r = check_ctx(ctx)) return r;
    if (!is_act_type(out_type)) return fail(LLMR_ERR_UNSUPPORTED, "output type %u not supported", out_type);
    if (int r = check_dim(dim)) return r;
    if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(LLMR_ERR_INVALID_ARG, "eps must be finite and >= 0");
    if (n_rows == 0) return ok();
    if (int r = check_rows(x, "x", x_stride, dim)) return r;
    if (int r = check_rows(out, "out", out_stride, dim)) return r;
    if (int r = check_vec(weight, "weight", !ln)) return r;
    if (ln && weight) return fail(LLMR_ERR_INVALID_ARG, "batch_layernorm has no affine weight (pass null)");
    if (int r = check_vec(mod_scale, "mod_scale", false)) return r;
    if (int r = check_vec(mod_shift, "mod_shift", false)) return r;
    if (int r = check_vec(mod_scale2, "mod_scale2", false)) return r;
    if (int r = check_vec(mod_shift2, "mod_shift2", false)) return r;
    llmr::RowNormArgs a{x, weight, mod_scale, mod_shift, out, x_stride, out_stride, n_rows, dim, eps,
                        mod_scale2, mod_shift2, split, (uint32_t)ctx->num_cus};
    return launched(llmr::launch_row_norm(a, ln, out_type, ctx->cur), ln ? "batch_layernorm" : "batch_rmsnorm");
}

}  // namespace

extern "C" {

int llmr_batch_rmsnorm(llmr_context* ctx, const float* x, uint32_t x_stride, const float* weight,
                       const float* mod_scale, const float* mod_shift, void* out, uint32_t out_type,
                       uint32_t out_stride, uint32_t dim, uint32_t n_rows, float eps) {
    return row_norm_common(ctx, false, x, x_stride, weight, mod_scale, mod_shift, out, out_type, out_stride, dim,
                           n_rows, eps);
}

int llmr_batch_layernorm(llmr_context* ctx, const float* x, uint32_t x_stride, const float* mod_scale,
                         const float* mod_shift, void* out, uint32_t out_type, uint32_t out_stride, uint32_t dim,
                         uint32_t n_rows, float eps) {
    return row_norm_common(ctx, true, x, x_stride, nullptr, mod_scale, mod_shift, out, out_type, out_stride, dim,
                           n_rows, eps);
}

int llmr_batch_layernorm_split(llmr_context* ctx, const float* x, uint32_t x_stride, const float* mod_scale,
                               const float* mod_shift, uint32_t split_row, const float* mod_scale2,
                               const float* mod_shift2, void* out, uint32_t out_type, uint32_t out_stride,
                               uint32_t dim, uint32_t n_rows, float eps) {
    if (split_row % 4 || split_row > n_rows)
        return fail(LLMR_ERR_INVALID_ARG, "split_row must be a multiple of 4 and <= n_rows (got %u of %u)", split_row,
                    n_rows);
    return row_norm_common(ctx, true, x, x_stride, nullptr, mod_scale, mod_shift, out, out_type, out_stride, dim,
                           n_rows, eps, split_row, mod_scale2, mod_shift2);
}

int llmr_qkv_heads(llmr_context* ctx, const float* qkv, uint32_t qkv_stride, uint32_t n_rows, uint32_t n_heads,
                   const float* q_norm, const float* k_norm, float eps, const float* rope_cos, const float* rope_sin,
                   void* q, void* k, void* v, uint32_t out_type, uint32_t seq_len, uint32_t row0) {
    if (int r = check_ctx(ctx)) return r;
    if (!is_act_type(out_type)) return fail(LLMR_ERR_UNSUPPORTED, "output type %u not supported", out_type);
    if (n_heads == 0 || n_heads > 1024) return fail(LLMR_ERR_INVALID_ARG, "n_heads must be in [1, 1024]");
    if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(LLMR_ERR_INVALID_ARG, "eps must be finite and >= 0");
    if ((uint64_t)row0 + n_rows > seq_len)
        return fail(LLMR_ERR_INVALID_ARG, "row0 + n_rows (%llu) > seq_len %u",
                    (unsigned long long)row0 + n_rows, seq_len);
    if (n_rows == 0) return ok();
    if (int r = check_rows(qkv, "qkv", qkv_stride, 3u * n_heads * 128u)) return r;
    if (int r = check_vec(q_norm, "q_norm", false)) return r;
    if (int r = check_vec(k_norm, "k_norm", false)) return r;
    if ((rope_cos == nullptr) != (rope_sin == nullptr))
        return fail(LLMR_ERR_INVALID_ARG, "rope_cos and rope_sin must both be given or both be null");
    if (int r = check_vec(rope_cos, "rope_cos", false)) return r;
    if (int r = check_vec(rope_sin, "rope_sin", false)) return r;
    if (int r = check_vec(q, "q", true)) return r;
    if (int r = check_vec(k, "k", true)) return r;
    if (int r = check_vec(v, "v", true)) return r;
    llmr::QkvHeadsArgs a{qkv, q_norm, k_norm, rope_cos, rope_sin, q, k, v, qkv_stride, n_rows, n_heads, seq_len,
                         row0, eps};
    return launched(llmr::launch_qkv_heads(a, out_type, ctx->cur), "qkv_heads");
}

int llmr_gated_residual(llmr_context* ctx, float* residual, uint32_t residual_stride, const float* input,
                        uint32_t input_stride, const float* norm_weight, const float* gate, uint32_t gate_mode,
                        uint32_t dim, uint32_t n_rows, float eps) {
    if (int r = check_ctx(ctx)) return r;
    if (gate_mode > LLMR_GATE_TANH) return fail(LLMR_ERR_INVALID_ARG, "unknown gate mode %u", gate_mode);
    if (int r = check_dim(dim)) return r;
    if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(LLMR_ERR_INVALID_ARG, "eps must be finite and >= 0");
    if (n_rows == 0) return ok();
    if (int r = check_rows(residual, "residual", residual_stride, dim)) return r;
    if (int r = check_rows(input, "input", input_stride, dim)) return r;
    if (int r = check_vec(norm_weight, "norm_weight", false)) return r;
    if (int r = check_vec(gate, "gate", gate_mode != LLMR_GATE_NONE)) return r;
    llmr::ResidualArgs a{residual, input, norm_weight, gate_mode == LLMR_GATE_NONE ? nullptr : gate,
                         residual_stride, input_stride, n_rows, dim, eps};
    a.grid_cus = (uint32_t)ctx->num_cus;
    return launched(llmr::launch_residual(a, gate_mode == LLMR_GATE_TANH, ctx->cur), "gated_residual");
}

int llmr_gated_residual_rmsnorm(llmr_context* ctx, float* residual, uint32_t residual_stride, const float* input,
                                uint32_t input_stride, const float* norm_weight, const float* gate, uint32_t gate_mode,
                                const float* next_weight, const float* next_scale, const float* next_shift, void* out,
                                uint32_t out_type, uint32_t out_stride, uint32_t dim, uint32_t n_rows, float eps,
                                float next_eps) {
    if (int r = check_ctx(ctx)) return r;
    if (gate_mode > LLMR_GATE_TANH) return fail(LLMR_ERR_INVALID_ARG, "unknown gate mode %u", gate_mode);
    if (!is_act_type(out_type)) return fail(LLMR_ERR_UNSUPPORTED, "output type %u not supported", out_type);
    if (int r = check_dim(dim)) return r;
    if (dim > 4096) return fail(LLMR_ERR_INVALID_ARG, "gated_residual_rmsnorm needs dim <= 4096 (got %u)", dim);
    if (!(eps >= 0.0f) || !std::isfinite(eps) || !(next_eps >= 0.0f) || !std::isfinite(next_eps))
        return fail(LLMR_ERR_INVALID_ARG, "eps and next_eps must be finite and >= 0");
    if (n_rows == 0) return ok();
    if (int r = check_rows(residual, "residual", residual_stride, dim)) return r;
    if (int r = check_rows(input, "input", input_stride, dim)) return r;
    if (int r = check_rows(out, "out", out_stride, dim)) return r;
    if (int r = check_vec(norm_weight, "norm_weight", false)) return r;
    if (int r = check_vec(gate, "gate", gate_mode != LLMR_GATE_NONE)) return r;
    if (int r = check_vec(next_weight, "next_weight", true)) return r;
    if (int r = check_vec(next_scale, "next_scale", false)) return r;
    if (int r = check_vec(next_shift, "next_shift", false)) return r;
    llmr::ResidualArgs a{residual, input, norm_weight, gate_mode == LLMR_GATE_NONE ? nullptr : gate,
                         residual_stride, input_stride, n_rows, dim, eps,
                         next_weight, next_scale, next_shift, out, out_stride, next_eps, (uint32_t)ctx->num_cus};
    return launched(llmr::launch_residual_norm(a, gate_mode == LLMR_GATE_TANH, out_type, ctx->cur),
                    "gated_residual_rmsnorm");
}

int llmr_activation(llmr_context* ctx, const float* src, uint32_t src_stride, uint32_t src_col, uint32_t src2_col,
                    void* dst, uint32_t dst_type, uint32_t dst_stride, uint32_t dst_col, uint32_t n_rows,
                    uint32_t n_cols, uint32_t act) {
    if (int r = check_ctx(ctx)) return r;
    if (!is_act_type(dst_type)) return fail(LLMR_ERR_UNSUPPORTED, "output type %u not supported", dst_type);
    if (act > LLMR_ACT_SILU_MUL) return fail(LLMR_ERR_INVALID_ARG, "unknown activation %u", act);
    if (n_cols % 4 || src_col % 4 || src2_col % 4 || dst_col % 4)
        return fail(LLMR_ERR_INVALID_ARG, "n_cols and column offsets must be multiples of 4");
    if (n_rows == 0 || n_cols == 0) return ok();
    const uint64_t src_w = (uint64_t)src_col + n_cols;
    const uint64_t src2_w = act == LLMR_ACT_SILU_MUL ? (uint64_t)src2_col + n_cols : 0;
    const uint64_t dst_w = (uint64_t)dst_col + n_cols;
    if (src_w > src_stride || src2_w > src_stride)
        return fail(LLMR_ERR_INVALID_ARG, "source columns exceed the row stride %u", src_stride);
    if (dst_w > dst_stride) return fail(LLMR_ERR_INVALID_ARG, "destination columns exceed the row stride %u", dst_stride);
    if (int r = check_rows(src, "src", src_stride, 0)) return r;
    if (int r = check_rows(dst, "dst", dst_stride, 0)) return r;
    if ((uint64_t)((n_cols / 4u + 255u) / 256u) * n_rows > 0x7fffffffull)
        return fail(LLMR_ERR_INVALID_ARG, "grid too large");
    llmr::ActColsArgs a{src, dst, src_stride, src_col, src2_col, dst_stride, dst_col, n_rows, n_cols};
    return launched(llmr::launch_act_cols(a, (int)act, dst_type, ctx->cur), "activation");
}

int llmr_timestep_embed(llmr_context* ctx, float* out, uint32_t dim, float timestep) {
    if (int r = check_ctx(ctx)) return r;
    if (dim == 0 || dim % 2) return fail(LLMR_ERR_INVALID_ARG, "dim must be even and > 0 (got %u)", dim);
    if (!out) return fail(LLMR_ERR_INVALID_ARG, "null output pointer");
    if (!std::isfinite(timestep)) return fail(LLMR_ERR_INVALID_ARG, "timestep must be finite");
    return launched(llmr::launch_timestep_embed(out, dim, timestep, ctx->cur), "timestep_embed");
}

static int patch_shape(uint32_t channels, uint32_t height, uint32_t width, uint32_t patch_size) {
    if (channels == 0 || height == 0 || width == 0 || patch_size == 0)
        return fail(LLMR_ERR_INVALID_ARG, "channels, height, width and patch_size must be > 0");
    if (height % patch_size || width % patch_size)
        return fail(LLMR_ERR_INVALID_ARG, "height and width must be multiples of patch_size");
    if ((uint64_t)channels * height * width > 0x7fffffffull)
        return fail(LLMR_ERR_INVALID_ARG, "latent too large");
    return LLMR_OK;
}

int llmr_patchify(llmr_context* ctx, const float* latent, void* out, uint32_t out_type, uint32_t channels,
                  uint32_t height, uint32_t width, uint32_t patch_size) {
    if (int r = check_ctx(ctx)) return r;
    if (!is_act_type(out_type)) return fail(LLMR_ERR_UNSUPPORTED, "output type %u not supported", out_type);
    if (int r = patch_shape(channels, height, width, patch_size)) return r;
    if (!latent || !out) return fail(LLMR_ERR_INVALID_ARG, "null pointer");
    return launched(llmr::launch_patchify(latent, out, out_type, channels, height, width, patch_size, ctx->cur),
                    "patchify");
}

int llmr_unpatchify(llmr_context* ctx, const float* patches, float* out, uint32_t channels, uint32_t height,
                    uint32_t width, uint32_t patch_size) {
    if (int r = check_ctx(ctx)) return r;
    if (int r = patch_shape(channels, height, width, patch_size)) return r;
    if (!patches || !out) return fail(LLMR_ERR_INVALID_ARG, "null pointer");
    return launched(llmr::launch_unpatchify(patches, out, channels, height, width, patch_size, ctx->cur),
                    "unpatchify");
}

int llmr_synth_q4k(llmr_context* ctx, void* out, uint64_t n_rows, uint32_t in_dim, uint64_t seed, uint64_t stream,
                   double std) {
    if (int r = check_ctx(ctx)) return r;
    if (in_dim == 0 || in_dim % 256) return fail(LLMR_ERR_INVALID_ARG, "in_dim must be a positive multiple of 256");
    if (!(std >= 0.0) || !std::isfinite(std)) return fail(LLMR_ERR_INVALID_ARG, "std must be finite and >= 0");
    if (n_rows == 0) return ok();
    if (!out || !aligned(out, 16)) return fail(LLMR_ERR_INVALID_ARG, "output must be non-null and 16-byte aligned");
    if (n_rows > (1ull << 33) / (in_dim / 256u))  // superblocks must fit the kernel's 2^31 x 4 waves
        return fail(LLMR_ERR_INVALID_ARG, "n_rows * in_dim / 256 too large");
    return launched(llmr::launch_synth_q4k(out, n_rows, in_dim, seed, stream, std, ctx->cur), "synth_q4k");
}

}  // extern "C"
