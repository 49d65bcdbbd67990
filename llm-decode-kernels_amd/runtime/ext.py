"""Loader of the MI355X decode-kernel library and the torch-facing op module.

Drop-in for the reference's ``runtime/ext.py`` (:9-20): ``load()`` returns an object with the six ops of the pybind
module ``decode_kernels`` (kernels/bindings.cpp:90-99) — same names, argument order, in-place/out-param conventions
and error behaviour (``RuntimeError`` for every TORCH_CHECK of kernels/bindings.cpp:18-88). Instead of a JIT nvcc
build it loads ``libdk_amd.so``, a hipcc-built C-ABI library (include/dk_amd.h), through ctypes; every op launches on
torch's current HIP stream, so the ops are capturable with ``torch.cuda.graph`` (a hipGraph on ROCm).

There is no CPU path: without the built library ``load()`` raises.
"""
import ctypes
import pathlib

import torch

PKG_DIR = pathlib.Path(__file__).resolve().parents[1]
LIB_PATH = PKG_DIR / "libdk_amd.so"
HEADER = PKG_DIR.parent / "include" / "dk_amd.h"

# Every exported entry point, with its ctypes signature (kept in the order of include/dk_amd.h).
_P, _I, _F, _Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
SIGNATURES = {
    "dk_last_error": ([], ctypes.c_char_p),
    "dk_runtime_version": ([], _I),
    "dk_gemv_w4a16": ([_I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _I, _P], _I),
    "dk_gemv_w4a16_rmsnorm": ([_I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _F, _P, _P, _I, _I, _I, _P], _I),
    "dk_gemv_w4a16_gate_up": ([_I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _F, _P, _P, _I, _I, _I, _P], _I),
    "dk_gemv_w4a16_qkv_rope": ([_I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I,
                                _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "dk_gemv_w4a16_attn": ([_I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _I, _I, _I,
                            _P], _I),
    "dk_gemv_f16": ([_I, _I, _I, _P, _P, _P, _I, _I, _P], _I),
    "dk_gemv_f16_rmsnorm": ([_I, _I, _I, _P, _P, _P, _P, _F, _P, _P, _I, _I, _P], _I),
    "dk_gemm_w4a16": ([_P, _P, _P, _P, _I, _I, _I, _I, _I, _P], _I),
    "dk_gemm_w4a16_workspace_bytes": ([_I, _I, _I, _I, _I], _Z),
    "dk_gemm_w4a16_ws": ([_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _Z, _P], _I),
    "dk_rope_append_rows": ([_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "dk_rmsnorm_rows_parts": ([_P, _P, _I, ctypes.c_longlong, _P, _P, _P, _I, _I, _F, _P], _I),
    "dk_rmsnorm_rows": ([_P, _P, _I, _P, _P, _P, _P, _I, _I, _F, _P], _I),
    "dk_attention_prefill": ([_P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P], _I),
    "dk_bw_read": ([_P, _Z, _P, _I, _I, _I, _I, _P], _I),
    "dk_paged_attention": ([_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P], _I),
    "dk_paged_attention_split": ([_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P], _I),
    "dk_paged_attention_noalloc": ([_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P], _I),
    "dk_paged_attention_noalloc_bytes": ([_I, _I, _I], _Z),
    "dk_attention_decode": ([_P, _P, _P, _I, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P],
                            _I),
    "dk_add_rmsnorm": ([_P, _P, _P, _P, _I, _F, _P], _I),
    "dk_swiglu": ([_P, _P, _I, _P], _I),
    "dk_rope_append": ([_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "dk_argmax_advance": ([_P, _I, _P, _P, _P], _I),
    "dk_argmax_advance_split": ([_P, _I, _P, _P, _P, _P], _I),
    "dk_quantize_w4": ([_P, _P, _P, _I, _I, _I, _I, _P], _I),
}

_EXT = None


def open_library(path=LIB_PATH):
    """dlopen the library and bind every entry point (no GPU needed). torch is imported first so the library resolves
    libamdhip64 to the HIP runtime torch already loaded (one runtime per process)."""
    if not pathlib.Path(path).exists():
        raise RuntimeError(f"{path} is not built: run `make -C llm-decode-kernels_amd/csrc` "
                           "(or __graft_entry__.build()); there is no CPU fallback")
    lib = ctypes.CDLL(str(path))
    for name, (argtypes, restype) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    return lib


def _check_cuda(t, name):
    if not (t.is_cuda and t.is_contiguous()):
        raise RuntimeError(f"{name} must be a contiguous CUDA tensor")


def _check_dtype(t, dtype, name):
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must be {dtype}, got {t.dtype}")


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


class DecodeKernels:
    """The op module. Every method validates like the reference binding, then calls one C entry point."""

    def __init__(self, lib):
        self.lib = lib

    def _call(self, fn, *args):
        rc = fn(*args)
        if rc != 0:
            raise RuntimeError(self.lib.dk_last_error().decode() or f"decode kernel error {rc}")

    # kernels/bindings.cpp:27-38
    def gemv_w4a16(self, stage, R, warps, pf, packed, sz, x, y, group):
        for t, n in ((packed, "packed"), (sz, "sz"), (x, "x"), (y, "y")):
            _check_cuda(t, n)
        N, K = packed.size(0), packed.size(1) * 8
        if K % 32 != 0 or K % group != 0:
            raise RuntimeError("K must be a multiple of 32 and of the group size")
        if group < 32:
            raise RuntimeError("group must be >= 32 (one uint4 never straddles a group)")
        if not (x.numel() == K and y.numel() == N and sz.size(0) == N and sz.size(1) == K // group):
            raise RuntimeError("gemv_w4a16: shape mismatch between packed, sz, x and y")
        _check_dtype(packed, torch.int32, "packed")
        for t, n in ((x, "x"), (y, "y"), (sz, "sz")):
            _check_dtype(t, torch.float16, n)
        self._call(self.lib.dk_gemv_w4a16, int(stage), int(R), int(warps), int(pf), packed.data_ptr(), sz.data_ptr(),
                   x.data_ptr(), y.data_ptr(), N, K, int(group), _stream(x))

    def _gemv_shape(self, packed, sz, y, K, group):
        N = packed.size(0)
        if packed.size(1) * 8 != K or y.numel() != N or sz.size(0) != N or sz.size(1) != K // group:
            raise RuntimeError("gemv: shape mismatch between packed, sz, x and y")
        _check_dtype(packed, torch.int32, "packed")
        _check_dtype(sz, torch.float16, "sz")
        _check_dtype(y, torch.float16, "y")
        return N

    # add_rmsnorm (kernels/bindings.cpp:64-72) fused into the gemv_w4a16 that follows it
    def gemv_w4a16_rmsnorm(self, stage, R, warps, pf, packed, sz, x, row, delta, norm_w, eps, x_out, y, group):
        for t, n in ((packed, "packed"), (sz, "sz"), (x, "x"), (norm_w, "norm_w"), (y, "y")):
            _check_cuda(t, n)
        K = norm_w.numel()
        N = self._gemv_shape(packed, sz, y, K, group)
        if row is None and x.numel() != K:
            raise RuntimeError("gemv_w4a16_rmsnorm: x must hold K values (or be a [*, K] table with row)")
        if row is not None and (x.dim() != 2 or x.size(1) != K or row.dtype != torch.int64 or delta is not None):
            raise RuntimeError("gemv_w4a16_rmsnorm: row needs an int64 index into a [*, K] x and no delta")
        for t, n in ((x, "x"), (norm_w, "norm_w")):
            _check_dtype(t, torch.float16, n)
        ptr = lambda t: None if t is None else t.data_ptr()
        for t, n in ((delta, "delta"), (x_out, "x_out"), (row, "row")):
            if t is not None:
                _check_cuda(t, n)
        for t, n in ((delta, "delta"), (x_out, "x_out")):
            if t is not None and (t.numel() != K or t.dtype != torch.float16):
                raise RuntimeError(f"gemv_w4a16_rmsnorm: {n} must be fp16 [K]")
        self._call(self.lib.dk_gemv_w4a16_rmsnorm, int(stage), int(R), int(warps), int(pf), packed.data_ptr(),
                   sz.data_ptr(), x.data_ptr(), ptr(row), ptr(delta), norm_w.data_ptr(), float(eps), ptr(x_out),
                   y.data_ptr(), N, K, int(group), _stream(x))

    # gemv_w4a16 of the interleaved gate|up rows followed by swiglu (kernels/bindings.cpp:27-38, 74-79), one launch;
    # the input is x itself (norm_w None) or the residual + RMSNorm of gemv_w4a16_rmsnorm
    def gemv_w4a16_gate_up(self, stage, R, warps, pf, packed, sz, x, row, delta, norm_w, eps, x_out, act, group):
        for t, n in ((packed, "packed"), (sz, "sz"), (x, "x"), (act, "act")):
            _check_cuda(t, n)
        K = packed.size(1) * 8
        N = packed.size(0)
        if N % 2 != 0 or act.numel() * 2 != N or sz.size(0) != N or sz.size(1) != K // group:
            raise RuntimeError("gemv_w4a16_gate_up: packed/sz need 2I interleaved rows and act I entries")
        _check_dtype(packed, torch.int32, "packed")
        _check_dtype(sz, torch.float16, "sz")
        _check_dtype(act, torch.float16, "act")
        _check_dtype(x, torch.float16, "x")
        if norm_w is None:
            if row is not None or delta is not None or x_out is not None or x.numel() != K:
                raise RuntimeError("gemv_w4a16_gate_up: without norm_w, x must hold K values and row/delta/x_out be None")
        else:
            _check_cuda(norm_w, "norm_w")
            _check_dtype(norm_w, torch.float16, "norm_w")
            if norm_w.numel() != K:
                raise RuntimeError("gemv_w4a16_gate_up: norm_w must hold K values")
            if row is None and x.numel() != K:
                raise RuntimeError("gemv_w4a16_gate_up: x must hold K values (or be a [*, K] table with row)")
            if row is not None and (x.dim() != 2 or x.size(1) != K or row.dtype != torch.int64 or delta is not None):
                raise RuntimeError("gemv_w4a16_gate_up: row needs an int64 index into a [*, K] x and no delta")
            for t, n in ((delta, "delta"), (x_out, "x_out"), (row, "row")):
                if t is not None:
                    _check_cuda(t, n)
            for t, n in ((delta, "delta"), (x_out, "x_out")):
                if t is not None and (t.numel() != K or t.dtype != torch.float16):
                    raise RuntimeError(f"gemv_w4a16_gate_up: {n} must be fp16 [K]")
        ptr = lambda t: None if t is None else t.data_ptr()
        self._call(self.lib.dk_gemv_w4a16_gate_up, int(stage), int(R), int(warps), int(pf), packed.data_ptr(),
                   sz.data_ptr(), x.data_ptr(), ptr(row), ptr(delta), ptr(norm_w), float(eps), ptr(x_out),
                   act.data_ptr(), N, K, int(group), _stream(x))

    # gemv_w4a16 of the qkv rows stored as per-head rotation pairs followed by rope_append (kernels/bindings.cpp
    # gemv_w4a16 then rope_append), one launch; the input is x itself (norm_w None) or the residual + RMSNorm input
    def gemv_w4a16_qkv_rope(self, stage, R, warps, pf, packed, sz, x, row, delta, norm_w, eps, x_out, qkv, cos_t,
                            sin_t, pos, bt, kc, vc, n_q, n_kv, group):
        """Shapes and dtypes are checked first, then that every tensor is a contiguous CUDA tensor, so no bad
        argument reaches the kernel."""
        what = "gemv_w4a16_qkv_rope"
        if kc.dim() != 4 or vc.shape != kc.shape or kc.size(1) != n_kv:
            raise RuntimeError(f"{what}: cache must be [pages, n_kv, P, head_dim] (kc and vc alike)")
        D = kc.size(3)
        K = packed.size(1) * 8
        N = (n_q + 2 * n_kv) * D
        if packed.dim() != 2 or packed.size(0) != N or qkv.numel() != N:
            raise RuntimeError(f"{what}: packed must hold (n_q + 2 n_kv) * head_dim rows and qkv as many values")
        if K % 32 != 0 or group < 32 or K % group != 0:
            raise RuntimeError(f"{what}: K must be a multiple of 32 and of the group size (>= 32)")
        self._gemv_shape(packed, sz, qkv, K, group)
        if cos_t.dim() != 2 or cos_t.size(1) * 2 != D or sin_t.shape != cos_t.shape:
            raise RuntimeError(f"{what}: cos_t and sin_t must both be [max_pos, head_dim / 2]")
        for t, n in ((x, "x"), (kc, "kc"), (vc, "vc")):
            _check_dtype(t, torch.float16, n)
        for t, n in ((cos_t, "cos_t"), (sin_t, "sin_t")):
            _check_dtype(t, torch.float32, n)
        for t, n in ((pos, "pos"), (bt, "bt")):
            _check_dtype(t, torch.int32, n)
        if pos.numel() < 1:
            raise RuntimeError(f"{what}: pos must hold the position (int32 [1])")
        if norm_w is None:
            if row is not None or delta is not None or x_out is not None or x.numel() != K:
                raise RuntimeError(f"{what}: without norm_w, x must hold K values and row/delta/x_out be None")
        else:
            if norm_w.numel() != K or norm_w.dtype != torch.float16:
                raise RuntimeError(f"{what}: norm_w must be fp16 [K]")
            if row is None and x.numel() != K:
                raise RuntimeError(f"{what}: x must hold K values (or be a [*, K] table with row)")
            if row is not None and (x.dim() != 2 or x.size(1) != K or row.dtype != torch.int64 or row.numel() != 1
                                    or delta is not None):
                raise RuntimeError(f"{what}: row needs one int64 index into a [*, K] x and no delta")
            for t, n in ((delta, "delta"), (x_out, "x_out")):
                if t is not None and (t.numel() != K or t.dtype != torch.float16):
                    raise RuntimeError(f"{what}: {n} must be fp16 [K]")
        for t, n in ((packed, "packed"), (sz, "sz"), (x, "x"), (qkv, "qkv"), (cos_t, "cos_t"), (sin_t, "sin_t"),
                     (pos, "pos"), (bt, "bt"), (kc, "kc"), (vc, "vc"), (row, "row"), (delta, "delta"),
                     (norm_w, "norm_w"), (x_out, "x_out")):
            if t is not None:
                _check_cuda(t, n)
        ptr = lambda t: None if t is None else t.data_ptr()
        self._call(self.lib.dk_gemv_w4a16_qkv_rope, int(stage), int(R), int(warps), int(pf), packed.data_ptr(),
                   sz.data_ptr(), x.data_ptr(), ptr(row), ptr(delta), ptr(norm_w), float(eps), ptr(x_out),
                   qkv.data_ptr(), cos_t.data_ptr(), sin_t.data_ptr(), pos.data_ptr(), bt.data_ptr(), kc.data_ptr(),
                   vc.data_ptr(), int(n_q), int(n_kv), D, kc.size(2), cos_t.size(0), kc.size(0), bt.numel(), K,
                   int(group), _stream(x))

    def _f16_shape(self, w, x, y, what):
        for t, n in ((w, "w"), (x, "x"), (y, "y")):
            _check_cuda(t, n)
            _check_dtype(t, torch.float16, n)
        if w.dim() != 2 or x.numel() != w.size(1) or y.numel() != w.size(0):
            raise RuntimeError(f"{what}: w must be [N, K], x [K] and y [N]")
        return w.size(0), w.size(1)

    # the fp16 LM head's torch.mm(x, W^T) (runtime/model.py:187) as a HIP GEMV
    def gemv_f16(self, R, warps, pf, w, x, y):
        N, Kd = self._f16_shape(w, x, y, "gemv_f16")
        self._call(self.lib.dk_gemv_f16, int(R), int(warps), int(pf), w.data_ptr(), x.data_ptr(), y.data_ptr(), N, Kd,
                   _stream(x))

    # add_rmsnorm (kernels/bindings.cpp:64-72) fused into the fp16 GEMV that follows it
    def gemv_f16_rmsnorm(self, R, warps, pf, w, x, delta, norm_w, eps, x_out, y):
        N, Kd = self._f16_shape(w, x, y, "gemv_f16_rmsnorm")
        _check_cuda(norm_w, "norm_w")
        for t, n in ((delta, "delta"), (norm_w, "norm_w"), (x_out, "x_out")):
            if t is not None:
                _check_cuda(t, n)
                if t.numel() != Kd or t.dtype != torch.float16:
                    raise RuntimeError(f"gemv_f16_rmsnorm: {n} must be fp16 [K]")
        ptr = lambda t: None if t is None else t.data_ptr()
        self._call(self.lib.dk_gemv_f16_rmsnorm, int(R), int(warps), int(pf), w.data_ptr(), x.data_ptr(), ptr(delta),
                   norm_w.data_ptr(), float(eps), ptr(x_out), y.data_ptr(), N, Kd, _stream(x))

    # prefill projections: Y = X . dequant(W)^T (epilogue 1: SwiGLU of interleaved gate/up pairs)
    def gemm_workspace_bytes(self, M, N, K, group, epilogue=0):
        """Bytes of split-K workspace dk_gemm_w4a16_ws uses for this shape (0: it does not split)."""
        return int(self.lib.dk_gemm_w4a16_workspace_bytes(int(M), int(N), int(K), int(group), int(epilogue)))

    def gemm_w4a16(self, packed, sz, x, y, group, epilogue=0, workspace=None):
        """y = x . dequant(W)^T (epilogue 1: SwiGLU of interleaved gate/up rows); `workspace` (a CUDA tensor of at
        least gemm_workspace_bytes bytes) lets the shapes that do not fill the CUs split K."""
        for t, n in ((packed, "packed"), (sz, "sz"), (x, "x"), (y, "y")):
            _check_cuda(t, n)
        N, K = packed.size(0), packed.size(1) * 8
        if x.dim() != 2 or x.size(1) != K:
            raise RuntimeError("gemm_w4a16: x must be [M, K]")
        M = x.size(0)
        if sz.size(0) != N or sz.size(1) != K // group or y.shape != (M, N // (1 + int(epilogue))):
            raise RuntimeError("gemm_w4a16: sz must be [N, K/G, 2] and y [M, N] (epilogue 1: [M, N/2])")
        _check_dtype(packed, torch.int32, "packed")
        for t, n in ((sz, "sz"), (x, "x"), (y, "y")):
            _check_dtype(t, torch.float16, n)
        if workspace is None:
            self._call(self.lib.dk_gemm_w4a16, packed.data_ptr(), sz.data_ptr(), x.data_ptr(), y.data_ptr(), M, N, K,
                       int(group), int(epilogue), _stream(x))
            return
        _check_cuda(workspace, "workspace")
        self._call(self.lib.dk_gemm_w4a16_ws, packed.data_ptr(), sz.data_ptr(), x.data_ptr(), y.data_ptr(), M, N, K,
                   int(group), int(epilogue), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
                   _stream(x))

    def gemm_w4a16_parts(self, packed, sz, x, group, workspace):
        """The split-K GEMM's fp32 partials alone (no reduce launch), left in `workspace`; returns them as a [S, M, N]
        float32 view of it. Only for shapes that split (gemm_workspace_bytes(M, N, K, group) > 0)."""
        for t, n in ((packed, "packed"), (sz, "sz"), (x, "x"), (workspace, "workspace")):
            _check_cuda(t, n)
        N, K = packed.size(0), packed.size(1) * 8
        if x.dim() != 2 or x.size(1) != K:
            raise RuntimeError("gemm_w4a16_parts: x must be [M, K]")
        M = x.size(0)
        if sz.size(0) != N or sz.size(1) != K // group:
            raise RuntimeError("gemm_w4a16_parts: sz must be [N, K/G, 2]")
        _check_dtype(packed, torch.int32, "packed")
        for t, n in ((sz, "sz"), (x, "x")):
            _check_dtype(t, torch.float16, n)
        need = self.gemm_workspace_bytes(M, N, K, group)
        self._call(self.lib.dk_gemm_w4a16_ws, packed.data_ptr(), sz.data_ptr(), x.data_ptr(), None, M, N, K,
                   int(group), 2, workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream(x))
        S = need // (M * N * 4)
        return workspace.view(torch.uint8)[:need].view(torch.float32).view(S, M, N)

    # prefill: residual + RMSNorm of M rows whose delta is split-K partials [S, M, H] (a view; rows contiguous)
    def rmsnorm_rows_parts(self, x_in, parts, w, x_out, out, eps):
        for t, n in ((x_in, "x_in"), (w, "w"), (x_out, "x_out"), (out, "out")):
            _check_cuda(t, n)
            _check_dtype(t, torch.float16, n)
        if not parts.is_cuda or parts.dtype != torch.float32 or parts.dim() != 3:
            raise RuntimeError("rmsnorm_rows_parts: parts must be a CUDA float32 [S, M, H] view")
        S, M, H = parts.shape
        if parts.stride(2) != 1 or parts.stride(1) != H or out.shape != (M, H) or x_in.shape != (M, H):
            raise RuntimeError("rmsnorm_rows_parts: parts [S, M, H] with contiguous rows; x_in, out [M, H]")
        self._call(self.lib.dk_rmsnorm_rows_parts, x_in.data_ptr(), parts.data_ptr(), S, parts.stride(0),
                   w.data_ptr(), x_out.data_ptr(), out.data_ptr(), M, H, float(eps), _stream(x_in))

    # prefill: rope_append over M token rows (row m at position *pos + m)
    def rope_append_rows(self, qkv, cos_t, sin_t, pos, bt, kc, vc, n_q, n_kv):
        for t, n in ((qkv, "qkv"), (cos_t, "cos_t"), (sin_t, "sin_t"), (pos, "pos"), (bt, "bt"), (kc, "kc"),
                     (vc, "vc")):
            _check_cuda(t, n)
        D = kc.size(3)
        if qkv.dim() != 2 or qkv.size(1) != (n_q + 2 * n_kv) * D:
            raise RuntimeError("rope_append_rows: qkv must be [M, (n_q + 2 n_kv) * D]")
        self._call(self.lib.dk_rope_append_rows, qkv.data_ptr(), cos_t.data_ptr(), sin_t.data_ptr(), pos.data_ptr(),
                   bt.data_ptr(), kc.data_ptr(), vc.data_ptr(), qkv.size(0), int(n_q), int(n_kv), D, kc.size(2),
                   cos_t.size(0), kc.size(0), bt.numel(), _stream(qkv))

    # prefill: residual + RMSNorm of M rows (rows: optional int64 gather index into x_in)
    def rmsnorm_rows(self, x_in, rows, delta, w, x_out, out, eps):
        for t, n in ((x_in, "x_in"), (w, "w"), (x_out, "x_out"), (out, "out")):
            _check_cuda(t, n)
            _check_dtype(t, torch.float16, n)
        M, H = out.shape
        if x_out.shape != (M, H) or w.numel() != H or x_in.size(-1) != H or (delta is not None and delta.shape != (M, H)):
            raise RuntimeError("rmsnorm_rows: x_out, out, delta [M, H], w [H], x_in [*, H]")
        if rows is not None and (rows.dtype != torch.int64 or rows.numel() != M):
            raise RuntimeError("rmsnorm_rows: rows must be int64 [M]")
        if rows is None and x_in.shape != (M, H):
            raise RuntimeError("rmsnorm_rows: without rows x_in must be [M, H]")
        ptr = lambda t: None if t is None else t.data_ptr()
        self._call(self.lib.dk_rmsnorm_rows, x_in.data_ptr(), ptr(rows), x_in.numel() // H, ptr(delta), w.data_ptr(),
                   x_out.data_ptr(), out.data_ptr(), M, H, float(eps), _stream(out))

    # prefill: causal attention of M rows over the paged cache
    def attention_prefill(self, qkv, pos, bt, kc, vc, n_q, n_kv, max_ctx, out):
        for t, n in ((qkv, "qkv"), (pos, "pos"), (bt, "bt"), (kc, "kc"), (vc, "vc"), (out, "out")):
            _check_cuda(t, n)
        D = kc.size(3)
        M = qkv.size(0)
        if qkv.dim() != 2 or qkv.size(1) != (n_q + 2 * n_kv) * D or out.shape != (M, n_q * D):
            raise RuntimeError("attention_prefill: qkv [M, (n_q + 2 n_kv) * D] and out [M, n_q * D]")
        self._call(self.lib.dk_attention_prefill, qkv.data_ptr(), pos.data_ptr(), bt.data_ptr(), bt.numel(),
                   kc.data_ptr(), vc.data_ptr(), kc.size(0), kc.size(2), int(n_q), int(n_kv), D, M, int(max_ctx),
                   out.data_ptr(), _stream(qkv))

    # kernels/bindings.cpp:40-43
    def bw_read(self, buf, sink, blocks, threads, unroll):
        """Read probe over buf with the caller's grid (blocks x threads, `unroll` 16-byte loads in flight per lane).
        A sink of at least blocks * threads / 64 32-bit words receives per-wave sums of the words read (slot
        b * threads / 64 + w), which add up to the 32-bit word sum of the buffer; a smaller sink is not written."""
        _check_cuda(buf, "buf")
        _check_cuda(sink, "sink")
        words = sink.numel() * sink.element_size() // 4
        if words < 1:
            raise RuntimeError("bw_read: sink must hold at least one 32-bit word")
        self._call(self.lib.dk_bw_read, buf.data_ptr(), buf.numel() * buf.element_size(), sink.data_ptr(), words,
                   int(blocks), int(threads), int(unroll), _stream(buf))

    # the checks of kernels/bindings.cpp:45-62 (head_dim generalised from 64 to {64, 128}) -> C arguments
    def _attention_args(self, q, kc, vc, bt, pos, part_size, o_part, m_part, l_part, out, version):
        for t, n in ((q, "q"), (kc, "kc"), (vc, "vc"), (bt, "bt"), (pos, "pos"), (out, "out"),
                     (o_part, "o_part"), (m_part, "m_part"), (l_part, "l_part")):
            _check_cuda(t, n)
        if kc.dim() != 4 or kc.size(3) not in (64, 128) or vc.shape != kc.shape:
            raise RuntimeError("cache must be [pages, n_kv, P, 64|128]")
        if bt.dtype != torch.int32 or pos.dtype != torch.int32:
            raise RuntimeError("bt and pos must be int32")
        for t, n in ((q, "q"), (kc, "kc"), (vc, "vc"), (out, "out")):
            _check_dtype(t, torch.float16, n)
        for t, n in ((o_part, "o_part"), (m_part, "m_part"), (l_part, "l_part")):
            _check_dtype(t, torch.float32, n)
        D = kc.size(3)
        n_q, n_kv, P = q.numel() // D, kc.size(1), kc.size(2)
        if n_q * D != q.numel() or n_q % n_kv != 0 or (n_q // n_kv) not in (1, 2, 4, 8):
            raise RuntimeError("heads-per-group must be 1/2/4/8")
        if part_size <= 0:
            raise RuntimeError("part_size must be > 0")
        if version not in (1, 2, 3, 4, 5):
            raise RuntimeError("attention version must be 1..5")
        max_splits = o_part.size(1)
        if not (o_part.size(0) == n_q and o_part.size(2) == D and m_part.size(0) == n_q and l_part.size(0) == n_q
                and m_part.size(1) == max_splits and l_part.size(1) == max_splits and out.numel() == n_q * D):
            raise RuntimeError("paged_attention: split buffers must be o [n_q, S, D], m/l [n_q, S], out [n_q, D]")
        return (int(version), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), pos.data_ptr(), n_q, n_kv, D,
                P, kc.size(0), bt.numel(), int(part_size), max_splits, o_part.data_ptr(), m_part.data_ptr(),
                l_part.data_ptr(), out.data_ptr(), _stream(q))

    # kernels/bindings.cpp:45-62 (head_dim generalised from 64 to {64, 128})
    def paged_attention(self, q, kc, vc, bt, pos, part_size, o_part, m_part, l_part, out, version=2):
        self._call(self.lib.dk_paged_attention,
                   *self._attention_args(q, kc, vc, bt, pos, part_size, o_part, m_part, l_part, out, version))

    # paged_attention's split kernel alone (no combine): with one live split it writes out, otherwise the partials
    # are left for gemv_w4a16_attn, the o projection that merges them in its prologue
    def paged_attention_split(self, q, kc, vc, bt, pos, part_size, o_part, m_part, l_part, out, version=5):
        self._call(self.lib.dk_paged_attention_split,
                   *self._attention_args(q, kc, vc, bt, pos, part_size, o_part, m_part, l_part, out, version))

    # the combine of paged_attention (kernels/paged_attention.cu:368-427) fused as the x prologue of gemv_w4a16 (the
    # o projection, runtime/model.py:220-222): y = W . combine(o_part, m_part, l_part), or W . attn with one live split
    def gemv_w4a16_attn(self, stage, R, warps, pf, packed, sz, o_part, m_part, l_part, attn, pos, bt, page, part_size,
                        max_pos, y, group):
        for t, n in ((packed, "packed"), (sz, "sz"), (o_part, "o_part"), (m_part, "m_part"), (l_part, "l_part"),
                     (attn, "attn"), (pos, "pos"), (bt, "bt"), (y, "y")):
            _check_cuda(t, n)
        for t, n in ((o_part, "o_part"), (m_part, "m_part"), (l_part, "l_part")):
            _check_dtype(t, torch.float32, n)
        _check_dtype(attn, torch.float16, "attn")
        if pos.dtype != torch.int32 or bt.dtype != torch.int32:
            raise RuntimeError("pos and bt must be int32")
        if o_part.dim() != 3:
            raise RuntimeError("gemv_w4a16_attn: o_part must be [n_q, S, D]")
        n_q, S, D = o_part.shape
        if m_part.shape != (n_q, S) or l_part.shape != (n_q, S) or attn.numel() != n_q * D:
            raise RuntimeError("gemv_w4a16_attn: split buffers must be o [n_q, S, D], m/l [n_q, S], attn [n_q * D]")
        K = n_q * D
        N = self._gemv_shape(packed, sz, y, K, group)
        self._call(self.lib.dk_gemv_w4a16_attn, int(stage), int(R), int(warps), int(pf), packed.data_ptr(),
                   sz.data_ptr(), o_part.data_ptr(), m_part.data_ptr(), l_part.data_ptr(), attn.data_ptr(),
                   pos.data_ptr(), bt.numel(), int(page), int(part_size), S, int(max_pos), n_q, D, y.data_ptr(), N, K,
                   int(group), _stream(y))

    # paged_attention with its split partials in the library's per-device scratch array (no caller buffers, no
    # allocation); calls that overlap on one GPU race
    def paged_attention_noalloc(self, q, kc, vc, bt, pos, part_size, max_splits, out, version=5):
        for t, n in ((q, "q"), (kc, "kc"), (vc, "vc"), (bt, "bt"), (pos, "pos"), (out, "out")):
            _check_cuda(t, n)
        if kc.dim() != 4 or kc.size(3) not in (64, 128) or vc.shape != kc.shape:
            raise RuntimeError("cache must be [pages, n_kv, P, 64|128]")
        if bt.dtype != torch.int32 or pos.dtype != torch.int32:
            raise RuntimeError("bt and pos must be int32")
        for t, n in ((q, "q"), (kc, "kc"), (vc, "vc"), (out, "out")):
            _check_dtype(t, torch.float16, n)
        D = kc.size(3)
        n_q, n_kv, P = q.numel() // D, kc.size(1), kc.size(2)
        if n_q * D != q.numel() or out.numel() != n_q * D:
            raise RuntimeError("paged_attention_noalloc: q and out must hold n_q * head_dim values")
        with torch.cuda.device(q.device):      # the scratch address is resolved on the current device
            self._call(self.lib.dk_paged_attention_noalloc, int(version), q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                       bt.data_ptr(), pos.data_ptr(), n_q, n_kv, D, P, kc.size(0), bt.numel(), int(part_size),
                       int(max_splits), out.data_ptr(), _stream(q))

    def paged_attention_noalloc_bytes(self, n_q, head_dim, max_splits):
        return int(self.lib.dk_paged_attention_noalloc_bytes(int(n_q), int(head_dim), int(max_splits)))

    # rope_append (kernels/bindings.cpp:81-88) + paged_attention (kernels/bindings.cpp:45-62) fused into one launch
    def attention_decode(self, qkv, cos_t, sin_t, pos, bt, kc, vc, n_q, n_kv, part_size, o_part, m_part, l_part,
                         out, impl=0):
        """impl: 0 or 1 = block kernel, 3 = lean MFMA kernel (pages >= 16 tokens, part_size a multiple of 16 up to
        512, 256 at head_dim 128); 2 (an MFMA kernel since removed) is rejected. The split kernel is followed by the
        combine kernel."""
        for t, n in ((qkv, "qkv"), (cos_t, "cos_t"), (sin_t, "sin_t"), (pos, "pos"), (bt, "bt"), (kc, "kc"),
                     (vc, "vc"), (o_part, "o_part"), (m_part, "m_part"), (l_part, "l_part"), (out, "out")):
            _check_cuda(t, n)
        if kc.dim() != 4 or kc.size(3) not in (64, 128) or vc.shape != kc.shape or kc.size(1) != n_kv:
            raise RuntimeError("cache must be [pages, n_kv, P, 64|128]")
        D = kc.size(3)
        if qkv.numel() != (n_q + 2 * n_kv) * D or cos_t.dim() != 2 or cos_t.size(1) != D // 2 \
                or sin_t.shape != cos_t.shape:
            raise RuntimeError("attention_decode: qkv must hold (n_q + 2 n_kv) * D values and cos/sin [max_pos, D/2]")
        for t, n in ((qkv, "qkv"), (kc, "kc"), (vc, "vc"), (out, "out")):
            _check_dtype(t, torch.float16, n)
        for t, n in ((cos_t, "cos_t"), (sin_t, "sin_t"), (o_part, "o_part"), (m_part, "m_part"), (l_part, "l_part")):
            _check_dtype(t, torch.float32, n)
        for t, n in ((pos, "pos"), (bt, "bt")):
            _check_dtype(t, torch.int32, n)
        if n_q % n_kv != 0 or (n_q // n_kv) not in (1, 2, 4, 8):
            raise RuntimeError("heads-per-group must be 1/2/4/8")
        max_splits = o_part.size(1)
        if not (o_part.size(0) == n_q and o_part.size(2) == D and m_part.shape == (n_q, max_splits)
                and l_part.shape == (n_q, max_splits) and out.numel() == n_q * D):
            raise RuntimeError("attention_decode: buffers must be o [n_q, S, D], m/l [n_q, S], out [n_q, D]")
        self._call(self.lib.dk_attention_decode, qkv.data_ptr(), cos_t.data_ptr(), sin_t.data_ptr(), cos_t.size(0),
                   pos.data_ptr(), bt.data_ptr(), bt.numel(), kc.data_ptr(), vc.data_ptr(), kc.size(0), kc.size(2),
                   int(n_q), int(n_kv), D, int(part_size), max_splits, int(impl), o_part.data_ptr(),
                   m_part.data_ptr(), l_part.data_ptr(), out.data_ptr(), _stream(qkv))

    # kernels/bindings.cpp:64-72
    def add_rmsnorm(self, x, delta, w, out, eps):
        _check_cuda(x, "x")
        _check_cuda(w, "w")
        _check_cuda(out, "out")
        if x.numel() % 8 != 0:
            raise RuntimeError("add_rmsnorm: numel must be a multiple of 8")
        if w.numel() != x.numel() or out.numel() != x.numel():
            raise RuntimeError("add_rmsnorm: x, w and out must have the same size")
        for t, n in ((x, "x"), (w, "w"), (out, "out")):
            _check_dtype(t, torch.float16, n)
        d = None
        if delta is not None:
            _check_cuda(delta, "delta")
            _check_dtype(delta, torch.float16, "delta")
            if delta.numel() != x.numel():
                raise RuntimeError("add_rmsnorm: delta must have the size of x")
            d = delta.data_ptr()
        self._call(self.lib.dk_add_rmsnorm, x.data_ptr(), d, w.data_ptr(), out.data_ptr(), x.numel(), float(eps),
                   _stream(x))

    # kernels/bindings.cpp:74-79
    def swiglu(self, gu, out):
        _check_cuda(gu, "gu")
        _check_cuda(out, "out")
        if not (out.numel() % 8 == 0 and gu.numel() == 2 * out.numel()):
            raise RuntimeError("swiglu: out.numel() % 8 == 0 and gu.numel() == 2 * out.numel() required")
        _check_dtype(gu, torch.float16, "gu")
        _check_dtype(out, torch.float16, "out")
        self._call(self.lib.dk_swiglu, gu.data_ptr(), out.data_ptr(), out.numel(), _stream(gu))

    # kernels/bindings.cpp:81-88 (head_dim generalised from 64 to {64, 128})
    def rope_append(self, qkv, cos_t, sin_t, pos, bt, kc, vc, n_q, n_kv):
        for t, n in ((qkv, "qkv"), (cos_t, "cos_t"), (sin_t, "sin_t"), (kc, "kc"), (vc, "vc"), (pos, "pos"),
                     (bt, "bt")):
            _check_cuda(t, n)
        if kc.dim() != 4 or kc.size(3) not in (64, 128) or vc.shape != kc.shape or kc.size(1) != n_kv:
            raise RuntimeError("cache must be [pages, n_kv, P, 64|128]")
        D = kc.size(3)
        if qkv.numel() != (n_q + 2 * n_kv) * D or cos_t.dim() != 2 or cos_t.size(1) != D // 2 \
                or sin_t.shape != cos_t.shape:
            raise RuntimeError("rope_append: qkv must hold (n_q + 2 n_kv) * D values and cos/sin [max_pos, D/2]")
        _check_dtype(qkv, torch.float16, "qkv")
        _check_dtype(cos_t, torch.float32, "cos_t")
        _check_dtype(sin_t, torch.float32, "sin_t")
        if bt.dtype != torch.int32 or pos.dtype != torch.int32:
            raise RuntimeError("bt and pos must be int32")
        self._call(self.lib.dk_rope_append, qkv.data_ptr(), cos_t.data_ptr(), sin_t.data_ptr(), pos.data_ptr(),
                   bt.data_ptr(), kc.data_ptr(), vc.data_ptr(), int(n_q), int(n_kv), D, kc.size(2), cos_t.size(0),
                   kc.size(0), bt.numel(), _stream(qkv))

    # runtime/model.py:232-233 (torch.argmax into tok, then pos += 1) as one launch
    def argmax_advance(self, logits, tok, pos=None):
        _check_cuda(logits, "logits")
        _check_cuda(tok, "tok")
        _check_dtype(logits, torch.float16, "logits")
        _check_dtype(tok, torch.int64, "tok")
        p = None
        if pos is not None:
            _check_cuda(pos, "pos")
            _check_dtype(pos, torch.int32, "pos")
            p = pos.data_ptr()
        self._call(self.lib.dk_argmax_advance, logits.data_ptr(), logits.numel(), tok.data_ptr(), p, _stream(logits))

    def argmax_advance_split(self, logits, tok, pos, work):
        """argmax_advance over ceil(V / 4096) workgroups that meet through `work` (int64 [2], zero before the first
        call, left zero by every call; one work buffer per stream of calls)."""
        _check_cuda(logits, "logits")
        _check_cuda(tok, "tok")
        _check_cuda(work, "work")
        _check_dtype(logits, torch.float16, "logits")
        _check_dtype(tok, torch.int64, "tok")
        _check_dtype(work, torch.int64, "work")
        if work.numel() != 2:
            raise RuntimeError("argmax_advance_split: work must be int64 [2]")
        p = None
        if pos is not None:
            _check_cuda(pos, "pos")
            _check_dtype(pos, torch.int32, "pos")
            p = pos.data_ptr()
        self._call(self.lib.dk_argmax_advance_split, logits.data_ptr(), logits.numel(), tok.data_ptr(), p,
                   work.data_ptr(), _stream(logits))

    # runtime/quant.py:42-48,100-124 on the GPU
    def quantize_w4(self, w, packed, sz, group, clip=False):
        for t, n in ((w, "w"), (packed, "packed"), (sz, "sz")):
            _check_cuda(t, n)
        N, K = w.shape
        if not (packed.shape == (N, K // 8) and sz.shape == (N, K // group, 2)):
            raise RuntimeError("quantize_w4: packed must be [N, K/8] int32 and sz [N, K/G, 2] fp16")
        _check_dtype(w, torch.float16, "w")
        _check_dtype(packed, torch.int32, "packed")
        _check_dtype(sz, torch.float16, "sz")
        self._call(self.lib.dk_quantize_w4, w.data_ptr(), packed.data_ptr(), sz.data_ptr(), N, K, int(group),
                   int(bool(clip)), _stream(w))


def load(verbose=False):
    """Load (once) and return the op module. Raises RuntimeError if the library is missing or not loadable."""
    global _EXT
    if _EXT is None:
        lib = open_library()
        _EXT = DecodeKernels(lib)
        if verbose:
            print(f"loaded {LIB_PATH} (HIP runtime {lib.dk_runtime_version()})")
    return _EXT
