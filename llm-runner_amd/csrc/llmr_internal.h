// llmr_internal.h - host-side launchers shared between the C-ABI layer
// (capi.hip) and the kernel translation units. Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmr {

// Launchers return hipSuccess or the launch error; argument validation is
// done by the C-ABI layer before they are called.
hipError_t launch_dequant_f32(const void* w, uint32_t wtype, uint32_t n_rows, uint32_t in_dim,
                              uint32_t row_offset, float* out, hipStream_t st);
hipError_t launch_dequant_operand_f16(const void* w, uint32_t wtype, uint32_t n_rows,
                                      uint32_t in_dim, uint32_t row_offset, uint16_t* out,
                                      hipStream_t st);

hipError_t launch_batch_matmul(const void* w, uint32_t wtype, const void* x, uint32_t xtype,
                               float* y, uint32_t out_dim, uint32_t in_dim, uint32_t seq_len,
                               uint32_t row_offset, int num_cus, hipStream_t st);

// SwiGLU of two Q8_0 GEMMs (batch_matmul_swiglu_q8). `ws` must hold
// swiglu_workspace_bytes(...) bytes (may be 0).
size_t swiglu_workspace_bytes(uint32_t wtype, uint32_t xtype, uint32_t out_dim, uint32_t in_dim,
                              uint32_t seq_len);
hipError_t launch_batch_matmul_swiglu(const void* wg, const void* wu, uint32_t wtype, const void* x,
                                      uint32_t xtype, float* y, uint32_t out_dim, uint32_t in_dim,
                                      uint32_t seq_len, int num_cus, void* ws, hipStream_t st);

hipError_t launch_flash_attention(const void* q, const void* k, const void* v, uint32_t xtype,
                                  float* o, uint32_t n_heads, uint32_t seq_len, float scale,
                                  hipStream_t st);

}  // namespace llmr
