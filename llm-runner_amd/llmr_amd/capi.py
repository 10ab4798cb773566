"""ctypes binding of the C-ABI in include/llmr_hip.h (libllmr_hip.so).

The library is built in-tree by llm-runner_amd/Makefile (or
__graft_entry__.build()). There is no fallback: if the library is missing or
fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import re

_PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(_PKG)                       # llm-runner_amd/
REPO = os.path.dirname(ROOT)
LIB_PATH = os.path.join(ROOT, "lib", "libllmr_hip.so")
HEADER_PATH = os.path.join(REPO, "include", "llmr_hip.h")

LLMR_OK = 0
LLMR_ERR_INVALID_ARG = 1
LLMR_ERR_UNSUPPORTED = 2
LLMR_ERR_HIP = 3
LLMR_ERR_NO_DEVICE = 4


class LlmrError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"llmr error {code}: {msg}")
        self.code = code


class BatchMatMulParams(ctypes.Structure):
    """BatchMatMulPC (dependencies/zimage.c3l/dit.c3:172-178)."""
    _fields_ = [("out_dim", ctypes.c_uint32), ("in_dim", ctypes.c_uint32),
                ("seq_len", ctypes.c_uint32), ("row_offset", ctypes.c_uint32)]


class FlashAttentionParams(ctypes.Structure):
    """FlashAttentionPC (dependencies/zimage.c3l/dit.c3:136-142)."""
    _fields_ = [("head_dim", ctypes.c_uint32), ("n_heads", ctypes.c_uint32),
                ("seq_len", ctypes.c_uint32), ("scale", ctypes.c_float)]


class MatmulJob(ctypes.Structure):
    """llmr_matmul_job: one GEMM of llmr_batch_matmul_multi."""
    _fields_ = [("weight", ctypes.c_void_p), ("input", ctypes.c_void_p), ("output", ctypes.c_void_p),
                ("gate", ctypes.c_void_p), ("output2", ctypes.c_void_p), ("seq_len", ctypes.c_uint32),
                ("row_offset", ctypes.c_uint32)]


class MatmulEpilogue(ctypes.Structure):
    """llmr_matmul_epilogue."""
    _fields_ = [("kind", ctypes.c_uint32), ("ldy", ctypes.c_uint32), ("split", ctypes.c_uint32),
                ("ldy2", ctypes.c_uint32), ("output2_type", ctypes.c_uint32)]


class NextWeightImage(ctypes.Structure):
    """llmr_next_weight_image: one weight image a call builds for a later call."""
    _fields_ = [("weight", ctypes.c_void_p), ("out_dim", ctypes.c_uint32), ("in_dim", ctypes.c_uint32),
                ("row_offset", ctypes.c_uint32), ("swiglu", ctypes.c_uint32), ("up_offset", ctypes.c_uint32),
                ("image", ctypes.c_void_p), ("image_bytes", ctypes.c_size_t)]


class NextWeightImages(ctypes.Structure):
    """llmr_next_weight_images: weight images of later GEMM groups (1 to 8)."""
    _fields_ = [("weight_type", ctypes.c_uint32), ("count", ctypes.c_uint32), ("image", NextWeightImage * 8)]


EPI_STORE, EPI_GATED_RESIDUAL, EPI_SPLIT_GELU, EPI_SPLIT_SWIGLU = 0, 1, 2, 3


class QkvHeadsJob(ctypes.Structure):
    """llmr_qkv_heads_job: one job's head norms and first sequence position."""
    _fields_ = [("q_norm", ctypes.c_void_p), ("k_norm", ctypes.c_void_p), ("row0", ctypes.c_uint32)]


class QkvHeadsOut(ctypes.Structure):
    """llmr_qkv_heads_out: the Q | K | V routing of llmr_batch_matmul_multi_qkv."""
    _fields_ = [("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
                ("out_type", ctypes.c_uint32), ("n_heads", ctypes.c_uint32), ("seq_len", ctypes.c_uint32),
                ("eps", ctypes.c_float), ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p),
                ("jobs", ctypes.POINTER(QkvHeadsJob))]


class GgufTensorInfo(ctypes.Structure):
    """llmr_gguf_tensor_info."""
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_uint32), ("n_dims", ctypes.c_uint32),
                ("ne", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64), ("data_size", ctypes.c_uint64),
                ("data", ctypes.c_void_p)]


class GgufKvInfo(ctypes.Structure):
    """llmr_gguf_kv_info."""
    _fields_ = [("key", ctypes.c_char_p), ("type", ctypes.c_uint32), ("array_type", ctypes.c_uint32),
                ("array_len", ctypes.c_uint64), ("data", ctypes.c_void_p), ("data_len", ctypes.c_uint64)]


class Lora(ctypes.Structure):
    """llmr_lora: a [rank, in_dim] and b [rows, rank] f32 device pointers, rank, scale."""
    _fields_ = [("a", ctypes.c_void_p), ("b", ctypes.c_void_p), ("rank", ctypes.c_uint32),
                ("scale", ctypes.c_float)]

_vp = ctypes.c_void_p
_u32 = ctypes.c_uint32
_SIGS = {
    "llmr_create_context": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(_vp)]),
    "llmr_destroy_context": (ctypes.c_int, [_vp]),
    "llmr_set_stream": (ctypes.c_int, [_vp, _vp]),
    "llmr_get_stream": (_vp, [_vp]),
    "llmr_last_error": (ctypes.c_char_p, []),
    "llmr_alloc": (ctypes.c_int, [_vp, ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "llmr_free": (ctypes.c_int, [_vp, _vp]),
    "llmr_upload": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_size_t]),
    "llmr_download": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_size_t]),
    "llmr_sync": (ctypes.c_int, [_vp]),
    "llmr_ggml_row_bytes": (ctypes.c_size_t, [_u32, _u32]),
    "llmr_dequant": (ctypes.c_int, [_vp, _vp, _u32, _u32, _u32, _u32, _vp]),
    "llmr_dequant_operand_f16": (ctypes.c_int, [_vp, _vp, _u32, _u32, _u32, _u32, _vp]),
    "llmr_batch_matmul": (ctypes.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _u32, _u32, _u32, _u32]),
    "llmr_batch_matmul_pc": (ctypes.c_int, [_vp, _vp, _u32, _vp, _u32, _vp,
                                            ctypes.POINTER(BatchMatMulParams)]),
    "llmr_batch_matmul_noalloc": (ctypes.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _u32, _u32, _u32, _u32]),
    "llmr_batch_matmul_multi": (ctypes.c_int, [_vp, _u32, _u32, _u32, _u32, ctypes.POINTER(MatmulJob), _u32,
                                               ctypes.POINTER(MatmulEpilogue)]),
    "llmr_batch_matmul_multi_images": (ctypes.c_int, [_vp, _u32, _u32, _u32, _u32, ctypes.POINTER(MatmulJob), _u32,
                                                      ctypes.POINTER(MatmulEpilogue), ctypes.POINTER(_vp),
                                                      ctypes.POINTER(NextWeightImages)]),
    "llmr_batch_matmul_multi_qkv": (ctypes.c_int, [_vp, _u32, _u32, _u32, _u32, ctypes.POINTER(MatmulJob), _u32,
                                                   ctypes.POINTER(MatmulEpilogue), ctypes.POINTER(QkvHeadsOut),
                                                   ctypes.POINTER(_vp), ctypes.POINTER(NextWeightImages)]),
    "llmr_weight_image_bytes": (ctypes.c_size_t, [_u32, _u32]),
    "llmr_swiglu_weight_image_bytes": (ctypes.c_size_t, [_u32, _u32]),
    "llmr_build_weight_image": (ctypes.c_int, [_vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp, ctypes.c_size_t]),
    "llmr_batch_matmul_swiglu": (ctypes.c_int, [_vp, _vp, _vp, _u32, _vp, _u32, _vp, _u32, _u32, _u32]),
    "llmr_batch_matmul_swiglu_pc": (ctypes.c_int, [_vp, _vp, _vp, _u32, _vp, _u32, _vp,
                                                   ctypes.POINTER(BatchMatMulParams)]),
    "llmr_flash_attention": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _u32,
                                            ctypes.c_float]),
    "llmr_flash_attention_rows": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _u32, _u32, _u32,
                                                 ctypes.c_float]),
    "llmr_flash_attention_pc": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _vp,
                                               ctypes.POINTER(FlashAttentionParams)]),
    "llmr_batch_rmsnorm": (ctypes.c_int, [_vp, _vp, _u32, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                          ctypes.c_float]),
    "llmr_batch_layernorm": (ctypes.c_int, [_vp, _vp, _u32, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                            ctypes.c_float]),
    "llmr_batch_layernorm_split": (ctypes.c_int, [_vp, _vp, _u32, _vp, _vp, _u32, _vp, _vp, _vp, _u32, _u32,
                                                  _u32, _u32, ctypes.c_float]),
    "llmr_qkv_heads": (ctypes.c_int, [_vp, _vp, _u32, _u32, _u32, _vp, _vp, ctypes.c_float, _vp, _vp,
                                      _vp, _vp, _vp, _u32, _u32, _u32]),
    "llmr_gated_residual": (ctypes.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _u32, _u32, _u32,
                                           ctypes.c_float]),
    "llmr_gated_residual_rmsnorm": (ctypes.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _u32, _vp, _vp, _vp, _vp,
                                                   _u32, _u32, _u32, _u32, ctypes.c_float, ctypes.c_float]),
    "llmr_activation": (ctypes.c_int, [_vp, _vp, _u32, _u32, _u32, _vp, _u32, _u32, _u32, _u32, _u32, _u32]),
    "llmr_timestep_embed": (ctypes.c_int, [_vp, _vp, _u32, ctypes.c_float]),
    "llmr_patchify": (ctypes.c_int, [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32]),
    "llmr_unpatchify": (ctypes.c_int, [_vp, _vp, _vp, _u32, _u32, _u32, _u32]),
    "llmr_synth_q4k": (ctypes.c_int, [_vp, _vp, ctypes.c_uint64, _u32, ctypes.c_uint64, ctypes.c_uint64,
                                      ctypes.c_double]),
    "llmr_lora_correction": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _u32, _u32, _u32, _u32]),
    "llmr_batch_matmul_lora": (ctypes.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _u32, _u32, _u32, _u32, _vp, _vp,
                                              _u32, _u32, _u32]),
    "llmr_q8_lora_merge": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, ctypes.c_float]),
    "llmr_gguf_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "llmr_gguf_close": (ctypes.c_int, [_vp]),
    "llmr_gguf_info": (ctypes.c_int, [_vp, ctypes.POINTER(_u32), ctypes.POINTER(ctypes.c_uint64),
                                      ctypes.POINTER(ctypes.c_uint64)]),
    "llmr_gguf_tensor": (ctypes.c_int, [_vp, ctypes.c_uint64, _vp]),
    "llmr_gguf_find_tensor": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]),
    "llmr_gguf_kv": (ctypes.c_int, [_vp, ctypes.c_uint64, _vp]),
    "llmr_gguf_find_kv": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]),
    "llmr_gguf_upload_tensor": (ctypes.c_int, [_vp, _vp, ctypes.c_uint64, _vp, ctypes.c_size_t]),
    "llmr_gguf_load_tensor": (ctypes.c_int, [_vp, _vp, ctypes.c_uint64, ctypes.POINTER(_vp)]),
}

# Activation and gate selectors of llmr_activation / llmr_gated_residual.
ACT_COPY, ACT_SILU, ACT_GELU_TANH, ACT_SILU_MUL = 0, 1, 2, 3
GATE_NONE, GATE_LINEAR, GATE_TANH = 0, 1, 2

_lib = None


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Names of every LLMR_API function declared in include/llmr_hip.h."""
    text = open(path).read()
    return re.findall(r"LLMR_API\s+[\w\s\*]+?\b(llmr_\w+)\s*\(", text)


def lib():
    """The loaded libllmr_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LlmrError(LLMR_ERR_NO_DEVICE,
                            f"{LIB_PATH} is not built; run `make -C llm-runner_amd` "
                            "or __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return (lib().llmr_last_error() or b"").decode()


def check(rc: int) -> None:
    if rc != LLMR_OK:
        raise LlmrError(rc, last_error())


class Context:
    """One device + one in-order stream (createContext, lib/vulkan/context.c3:73)."""

    def __init__(self, device: int = 0):
        self._h = _vp()
        check(lib().llmr_create_context(device, ctypes.byref(self._h)))

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        if self._h:
            lib().llmr_destroy_context(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream_ptr: int | None) -> None:
        check(lib().llmr_set_stream(self._h, stream_ptr or None))  # 0/None: HIP null stream

    def stream(self) -> int:
        return lib().llmr_get_stream(self._h) or 0

    def sync(self) -> None:
        check(lib().llmr_sync(self._h))

    def dequant(self, w_ptr: int, wtype: int, n_rows: int, in_dim: int, row_offset: int,
                out_ptr: int) -> None:
        check(lib().llmr_dequant(self._h, w_ptr, wtype, n_rows, in_dim, row_offset, out_ptr))

    def dequant_operand_f16(self, w_ptr: int, wtype: int, n_rows: int, in_dim: int,
                            row_offset: int, out_ptr: int) -> None:
        check(lib().llmr_dequant_operand_f16(self._h, w_ptr, wtype, n_rows, in_dim, row_offset,
                                             out_ptr))

    def batch_matmul(self, w_ptr: int, wtype: int, x_ptr: int, xtype: int, y_ptr: int,
                     out_dim: int, in_dim: int, seq_len: int, row_offset: int = 0) -> None:
        check(lib().llmr_batch_matmul(self._h, w_ptr, wtype, x_ptr, xtype, y_ptr, out_dim, in_dim,
                                      seq_len, row_offset))

    def batch_matmul_noalloc(self, w_ptr: int, wtype: int, x_ptr: int, xtype: int, y_ptr: int,
                             out_dim: int, in_dim: int, seq_len: int, row_offset: int = 0) -> None:
        check(lib().llmr_batch_matmul_noalloc(self._h, w_ptr, wtype, x_ptr, xtype, y_ptr, out_dim, in_dim,
                                              seq_len, row_offset))

    def batch_matmul_multi(self, wtype: int, xtype: int, out_dim: int, in_dim: int, jobs, epilogue=None) -> None:
        """jobs: sequence of MatmulJob; epilogue: MatmulEpilogue or None (plain store)."""
        arr = (MatmulJob * len(jobs))(*jobs)
        check(lib().llmr_batch_matmul_multi(self._h, wtype, xtype, out_dim, in_dim, arr, len(jobs),
                                            ctypes.byref(epilogue) if epilogue is not None else None))

    def batch_matmul_multi_images(self, wtype: int, xtype: int, out_dim: int, in_dim: int, jobs, epilogue,
                                  images=None, next_images: NextWeightImages | None = None) -> None:
        """As batch_matmul_multi with images[i] = device pointer of job i's weight
        image (or None), and the next group's images built (or None)."""
        arr = (MatmulJob * len(jobs))(*jobs)
        imgs = (_vp * len(jobs))(*images) if images is not None else None
        check(lib().llmr_batch_matmul_multi_images(self._h, wtype, xtype, out_dim, in_dim, arr, len(jobs),
                                                   ctypes.byref(epilogue) if epilogue is not None else None, imgs,
                                                   ctypes.byref(next_images) if next_images is not None else None))

    def batch_matmul_multi_qkv(self, wtype: int, xtype: int, out_dim: int, in_dim: int, jobs, epilogue,
                               heads: QkvHeadsOut, head_jobs=None, images=None,
                               next_images: NextWeightImages | None = None) -> None:
        """As batch_matmul_multi_images with the Q | K | V columns routed by
        `heads`; head_jobs: one QkvHeadsJob per job, or None."""
        arr = (MatmulJob * len(jobs))(*jobs)
        imgs = (_vp * len(jobs))(*images) if images is not None else None
        hj = (QkvHeadsJob * len(jobs))(*head_jobs) if head_jobs is not None else None
        h = QkvHeadsOut(heads.q, heads.k, heads.v, heads.out_type, heads.n_heads, heads.seq_len, heads.eps,
                        heads.rope_cos, heads.rope_sin, hj)
        check(lib().llmr_batch_matmul_multi_qkv(self._h, wtype, xtype, out_dim, in_dim, arr, len(jobs),
                                                ctypes.byref(epilogue) if epilogue is not None else None,
                                                ctypes.byref(h), imgs,
                                                ctypes.byref(next_images) if next_images is not None else None))

    def build_weight_image(self, w_ptr: int, wtype: int, xtype: int, out_dim: int, in_dim: int, row_offset: int,
                           img_ptr: int, img_bytes: int) -> None:
        check(lib().llmr_build_weight_image(self._h, w_ptr, wtype, xtype, out_dim, in_dim, row_offset, img_ptr,
                                            img_bytes))

    def batch_matmul_swiglu(self, wg_ptr: int, wu_ptr: int, wtype: int, x_ptr: int, xtype: int,
                            y_ptr: int, out_dim: int, in_dim: int, seq_len: int) -> None:
        check(lib().llmr_batch_matmul_swiglu(self._h, wg_ptr, wu_ptr, wtype, x_ptr, xtype, y_ptr,
                                             out_dim, in_dim, seq_len))

    def flash_attention_rows(self, q_ptr: int, k_ptr: int, v_ptr: int, xtype: int, o_ptr: int, otype: int,
                             ostride: int, head_dim: int, n_heads: int, seq_len: int, scale: float) -> None:
        check(lib().llmr_flash_attention_rows(self._h, q_ptr, k_ptr, v_ptr, xtype, o_ptr, otype, ostride, head_dim,
                                              n_heads, seq_len, scale))

    def flash_attention(self, q_ptr: int, k_ptr: int, v_ptr: int, xtype: int, o_ptr: int,
                        head_dim: int, n_heads: int, seq_len: int, scale: float) -> None:
        check(lib().llmr_flash_attention(self._h, q_ptr, k_ptr, v_ptr, xtype, o_ptr, head_dim,
                                         n_heads, seq_len, float(scale)))

    # --- block glue (pointers are device addresses, strides in elements) ---

    def batch_rmsnorm(self, x, x_stride, w, scale, shift, out, otype, out_stride, dim, rows, eps):
        check(lib().llmr_batch_rmsnorm(self._h, x, x_stride, w, scale, shift, out, otype, out_stride, dim,
                                       rows, float(eps)))

    def batch_layernorm(self, x, x_stride, scale, shift, out, otype, out_stride, dim, rows, eps):
        check(lib().llmr_batch_layernorm(self._h, x, x_stride, scale, shift, out, otype, out_stride, dim,
                                         rows, float(eps)))

    def batch_layernorm_split(self, x, x_stride, scale, shift, split_row, scale2, shift2, out, otype, out_stride,
                              dim, rows, eps):
        check(lib().llmr_batch_layernorm_split(self._h, x, x_stride, scale, shift, split_row, scale2, shift2, out,
                                               otype, out_stride, dim, rows, float(eps)))

    def qkv_heads(self, qkv, qkv_stride, rows, n_heads, q_norm, k_norm, eps, cos_t, sin_t, q, k, v, otype,
                  seq_len, row0):
        check(lib().llmr_qkv_heads(self._h, qkv, qkv_stride, rows, n_heads, q_norm, k_norm, float(eps), cos_t,
                                   sin_t, q, k, v, otype, seq_len, row0))

    def gated_residual(self, h, h_stride, x, x_stride, norm_w, gate, mode, dim, rows, eps):
        check(lib().llmr_gated_residual(self._h, h, h_stride, x, x_stride, norm_w, gate, mode, dim, rows,
                                        float(eps)))

    def gated_residual_rmsnorm(self, h, h_stride, x, x_stride, norm_w, gate, mode, next_w, next_scale, next_shift,
                               out, otype, out_stride, dim, rows, eps, next_eps):
        check(lib().llmr_gated_residual_rmsnorm(self._h, h, h_stride, x, x_stride, norm_w, gate, mode, next_w,
                                                next_scale, next_shift, out, otype, out_stride, dim, rows,
                                                float(eps), float(next_eps)))

    def activation(self, src, src_stride, src_col, src2_col, dst, dtype, dst_stride, dst_col, rows, cols, act):
        check(lib().llmr_activation(self._h, src, src_stride, src_col, src2_col, dst, dtype, dst_stride,
                                    dst_col, rows, cols, act))

    def timestep_embed(self, out, dim, t):
        check(lib().llmr_timestep_embed(self._h, out, dim, float(t)))

    def patchify(self, latent, out, otype, C, H, W, ps):
        check(lib().llmr_patchify(self._h, latent, out, otype, C, H, W, ps))

    def unpatchify(self, patches, out, C, H, W, ps):
        check(lib().llmr_unpatchify(self._h, patches, out, C, H, W, ps))

    def synth_q4k(self, out, n_rows, in_dim, seed, stream, std):
        check(lib().llmr_synth_q4k(self._h, out, n_rows, in_dim, seed, stream, float(std)))

    def lora_correction(self, lora: "Lora | None", scratch: int, x_ptr: int, xtype: int, y_ptr: int,
                        in_dim: int, out_dim: int, seq_len: int, b_rows: int = 0, row_offset: int = 0,
                        weight_row_offset: int = 0) -> None:
        check(lib().llmr_lora_correction(self._h, ctypes.byref(lora) if lora is not None else None, scratch,
                                         x_ptr, xtype, y_ptr, in_dim, out_dim, seq_len, b_rows, row_offset,
                                         weight_row_offset))

    def batch_matmul_lora(self, w_ptr: int, wtype: int, x_ptr: int, xtype: int, y_ptr: int, out_dim: int,
                          in_dim: int, seq_len: int, row_offset: int, lora: "Lora | None", scratch: int,
                          b_rows: int = 0, lora_row_offset: int = 0, lora_weight_row_offset: int = 0) -> None:
        check(lib().llmr_batch_matmul_lora(self._h, w_ptr, wtype, x_ptr, xtype, y_ptr, out_dim, in_dim, seq_len,
                                           row_offset, ctypes.byref(lora) if lora is not None else None, scratch,
                                           b_rows, lora_row_offset, lora_weight_row_offset))

    def q8_lora_merge(self, w_ptr: int, a_ptr: int, b_ptr: int, in_dim: int, b_rows: int, dst_row_offset: int,
                      rank: int, scale: float) -> None:
        check(lib().llmr_q8_lora_merge(self._h, w_ptr, a_ptr, b_ptr, in_dim, b_rows, dst_row_offset, rank,
                                       float(scale)))
