"""Loader for the gfx950 shared library and the PyTorch custom ops over it.

The library (`_lib/libgpa_mi355x.so`, built by `gpa-vggt_amd/build.py`)
exports the plain C ABI declared in `include/gpa_mi355x.h`.  This module
binds it with ctypes *after* importing torch, so the library resolves
`libamdhip64.so.7` to the HIP runtime torch already loaded, and registers
two custom ops:

    gpa::sim_argmax(Tensor a, Tensor b) -> (Tensor max_f32, Tensor idx_i64)
    gpa::attn_keybias(Tensor q, Tensor k, Tensor v, Tensor? bias,
                      float sm_scale, bool return_lse) -> (Tensor o, Tensor lse)
    gpa::merge_heads(Tensor t, Tensor offsets, Tensor tokens, int slots,
                     bool mean) -> (Tensor out, Tensor size, Tensor log_size)
    gpa::lse_combine(Tensor out_a, Tensor lse_a, Tensor out_b, Tensor lse_b,
                     int frames) -> Tensor y              (bf16 or fp16)
    gpa::qk_norm_rope(Tensor qkv, Tensor ln_w, Tensor ln_b, float eps,
                      Tensor? pos, Tensor? rope_cs, int heads, bool q_f32,
                      bool k_f32) -> (Tensor q, Tensor k)
    gpa::pool_shared(Tensor k, Tensor v, int frames, int pts, int grid_h,
                     int grid_w, int kp, bool want_assign)
                     -> (Tensor pk, Tensor pv, Tensor size, Tensor assign)

All launch on torch's current stream of the input's device.  There is no
fallback: a missing library or a non-GPU tensor raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import Optional, Tuple

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libgpa_mi355x.so"
ABI_VERSION = 15

GPA_OK = 0
GPA_E_INVALID = -1
GPA_E_UNSUPPORTED = -2
GPA_E_WORKSPACE = -3
GPA_E_LAUNCH = -4

GPA_BIAS_NONE = 0
GPA_BIAS_F32 = 1
GPA_BIAS_BF16 = 2
GPA_BIAS_F16 = 3

# Bytes of the static device scratch behind gpa_attn_keybias_bf16_noalloc
# (GPA_ATTN_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 32 << 20

GPA_DTYPE_F32 = 0
GPA_DTYPE_BF16 = 1
GPA_DTYPE_F16 = 2
_DTYPE_CODES = {torch.float32: GPA_DTYPE_F32, torch.bfloat16: GPA_DTYPE_BF16,
                          torch.float16: GPA_DTYPE_F16}
GPA_MERGE_SUM = 0
GPA_MERGE_MEAN = 1

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


class NativeLibraryError(RuntimeError):
    """The gfx950 library is missing, stale or failed to load."""


def _bind(lib: ctypes.CDLL) -> None:
    lib.gpa_abi_version.restype = ctypes.c_int
    lib.gpa_abi_version.argtypes = []
    lib.gpa_last_error.restype = ctypes.c_char_p
    lib.gpa_last_error.argtypes = []
    lib.gpa_sim_argmax_workspace_bytes.restype = ctypes.c_size_t
    lib.gpa_sim_argmax_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64]
    lib.gpa_sim_argmax_bf16.restype = ctypes.c_int
    lib.gpa_sim_argmax_bf16.argtypes = [
        _vp, _vp, _vp, ctypes.c_int, _vp,  # a, b, out_max, max_dtype, out_idx
        _i64, _i64, _i64, _i64,        # B, M, N, D
        _i64, _i64, _i64, _i64,        # a_sb, a_sm, b_sb, b_sn
        _i64, _i64,                    # omax_sb, oidx_sb
        _vp, ctypes.c_size_t, _vp,     # workspace, workspace_bytes, stream
    ]
    lib.gpa_sim_argmax_f16.restype = ctypes.c_int
    lib.gpa_sim_argmax_f16.argtypes = lib.gpa_sim_argmax_bf16.argtypes
    lib.gpa_attn_keybias_workspace_bytes.restype = ctypes.c_size_t
    lib.gpa_attn_keybias_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64]
    lib.gpa_attn_keybias_bf16.restype = ctypes.c_int
    lib.gpa_attn_keybias_bf16.argtypes = [
        _vp, _vp, _vp,                 # q, k, v
        _vp, ctypes.c_int,             # bias, bias_kind
        _i64, _i64, _i64,              # bias strides (b, h, n)
        _vp, _vp,                      # o, lse
        _i64, _i64, _i64, _i64, _i64,  # B, H, M, N, D
        _i64, _i64, _i64,              # q strides
        _i64, _i64, _i64,              # k strides
        _i64, _i64, _i64,              # v strides
        _i64, _i64, _i64,              # o strides
        _i64, _i64,                    # lse strides
        _vp, ctypes.c_size_t,          # workspace, workspace_bytes
        ctypes.c_float, _vp,           # sm_scale, stream
    ]
    lib.gpa_attn_keybias_f16.restype = ctypes.c_int
    lib.gpa_attn_keybias_f16.argtypes = lib.gpa_attn_keybias_bf16.argtypes
    lib.gpa_attn_keybias_bf16_noalloc.restype = ctypes.c_int
    lib.gpa_attn_keybias_bf16_noalloc.argtypes = (
        lib.gpa_attn_keybias_bf16.argtypes[:-4] + [ctypes.c_float, _vp])   # no workspace
    lib.gpa_lse_combine_bf16.restype = ctypes.c_int
    lib.gpa_lse_combine_bf16.argtypes = [_vp] * 5 + [_i64] * 5 + [_i64] * 16 + [_i64] * 3 + [_vp]
    lib.gpa_lse_combine_f16.restype = ctypes.c_int
    lib.gpa_lse_combine_f16.argtypes = lib.gpa_lse_combine_bf16.argtypes
    lib.gpa_qk_norm_rope_bf16.restype = ctypes.c_int
    lib.gpa_qk_norm_rope_bf16.argtypes = [
        _vp, _i64, _i64, _i64, _i64,   # qkv, B, N, H, D
        _i64, _i64, _i64,              # qkv_sb, qkv_sn, k_offset
        _vp, _vp, ctypes.c_float,      # ln_weight, ln_bias, eps
        _vp, _i64, _vp, _i64,          # pos, period, rope_cs, npos
        _vp, ctypes.c_int, _vp, ctypes.c_int,  # q_out, q_dtype, k_out, k_dtype
        _vp,                           # stream
    ]
    lib.gpa_qk_norm_rope_f16.restype = ctypes.c_int
    lib.gpa_qk_norm_rope_f16.argtypes = lib.gpa_qk_norm_rope_bf16.argtypes
    lib.gpa_pool_shared_bf16.restype = ctypes.c_int
    lib.gpa_pool_shared_bf16.argtypes = [
        _vp, _vp, _vp, _vp, _vp, _vp,  # k, v, pooled_k, pooled_v, size, assign
        _i64, _i64, _i64, _i64, _i64,  # B, H, S, P, pts
        _i64, _i64, _i64, _i64,        # grid_h, grid_w, kp, D
        _i64, _i64, _i64, _i64, _i64, _i64,  # k strides, v strides
        _vp,                           # stream
    ]
    lib.gpa_pool_shared_f16.restype = ctypes.c_int
    lib.gpa_pool_shared_f16.argtypes = lib.gpa_pool_shared_bf16.argtypes
    lib.gpa_merge_metric_bf16.restype = ctypes.c_int
    lib.gpa_merge_metric_bf16.argtypes = [
        _vp, ctypes.c_int,             # metric, metric dtype
        _i64, _i64, _i64, _i64, _i64,  # B, N, C, metric strides (b, n)
        _vp, _i64, _vp, ctypes.c_int,  # proj, P, order, norm_mode
        _vp, _vp,                      # out, stream
    ]
    lib.gpa_residual_layernorm_bf16.restype = ctypes.c_int
    lib.gpa_residual_layernorm_bf16.argtypes = [
        _vp, _vp, _vp, _vp, _vp, ctypes.c_float,  # x, y, gamma, weight, bias, eps
        _i64, _i64, _i64, _i64,        # rows, C, x_sn, y_sn
        _vp, _i64, _vp, _i64,          # h_out, h_sn, ln_out, ln_sn
        _vp,                           # stream
    ]
    lib.gpa_residual_layernorm_f16.restype = ctypes.c_int
    lib.gpa_residual_layernorm_f16.argtypes = lib.gpa_residual_layernorm_bf16.argtypes
    lib.gpa_merge_heads.restype = ctypes.c_int
    lib.gpa_merge_heads.argtypes = [
        _vp, ctypes.c_int, _vp,        # t, dtype, out
        _vp, _vp,                      # offsets, tokens
        _i64, _i64, _i64, _i64, _i64,  # B, H, N, S, D
        _i64, _i64, _i64,              # t strides (b, h, n)
        _i64, _i64, _i64,              # out strides (b, h, s)
        ctypes.c_int, _vp, _vp, _vp,   # mode, size_out, log_size_out, stream
    ]


def lib() -> ctypes.CDLL:
    """The loaded library (loaded on first use)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NativeLibraryError(
                    f"{LIB_PATH} is not built; run `python gpa-vggt_amd/build.py` "
                    "(hipcc, gfx950) before using the merging ops")
            handle = ctypes.CDLL(str(LIB_PATH))
            _bind(handle)
            ver = handle.gpa_abi_version()
            if ver != ABI_VERSION:
                raise NativeLibraryError(
                    f"{LIB_PATH} has ABI version {ver}, expected {ABI_VERSION}; rebuild it")
            _lib = handle
    return _lib


def exported_symbols() -> Tuple[str, ...]:
    return ("gpa_abi_version", "gpa_last_error", "gpa_sim_argmax_workspace_bytes",
            "gpa_sim_argmax_bf16", "gpa_attn_keybias_workspace_bytes", "gpa_attn_keybias_bf16",
            "gpa_merge_heads", "gpa_lse_combine_bf16", "gpa_qk_norm_rope_bf16",
            "gpa_pool_shared_bf16", "gpa_merge_metric_bf16", "gpa_sim_argmax_f16",
            "gpa_attn_keybias_f16", "gpa_residual_layernorm_bf16",
            "gpa_attn_keybias_bf16_noalloc", "gpa_lse_combine_f16", "gpa_qk_norm_rope_f16",
            "gpa_residual_layernorm_f16", "gpa_pool_shared_f16")


def _check(rc: int, what: str) -> None:
    if rc == GPA_OK:
        return
    msg = (lib().gpa_last_error() or b"").decode(errors="replace")
    if rc in (GPA_E_INVALID, GPA_E_WORKSPACE):
        raise ValueError(f"{what}: {msg}")
    if rc == GPA_E_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (code {rc})")


def _require_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError("the gfx950 merging kernels need GPU tensors, got device "
                             f"{t.device}")
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _st(t: torch.Tensor, dim: int) -> int:
    """Stride of `dim`, or 0 for a size-1 dimension (whose stride is arbitrary)."""
    return t.stride(dim) if t.shape[dim] > 1 else 0


def _rs(t: torch.Tensor, dim: int) -> int:
    """Row stride of `dim`; a single row reports its own width (stride unused)."""
    return t.stride(dim) if t.shape[dim] > 1 else t.shape[-1]


def _rows_ok(t: torch.Tensor, align_elems: int) -> bool:
    """Unit inner stride, other strides multiples of `align_elems`, aligned base."""
    if t.stride(-1) != 1:
        return False
    if t.data_ptr() % (t.element_size() * align_elems) != 0:
        return False
    return all(s % align_elems == 0 for s, n in zip(t.stride()[:-1], t.shape[:-1]) if n > 1)


# --------------------------------------------------------------------------
# gpa::sim_argmax
# --------------------------------------------------------------------------

@torch.library.custom_op("gpa::sim_argmax", mutates_args=())
def sim_argmax(a: torch.Tensor, b: torch.Tensor,
               max_in_input_dtype: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Row max and lowest-index argmax (int64) of a @ b^T; a and b both bf16
    or both fp16.  The max is fp32, or a's dtype (the fp32 max rounded to
    nearest even, written by the kernel) with max_in_input_dtype."""
    dev = _require_gpu(a, b)
    if a.dtype != b.dtype or a.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"gpa::sim_argmax takes two bf16 or two fp16 inputs, got "
                         f"{a.dtype}/{b.dtype}")
    if a.dim() != 3 or b.dim() != 3 or a.shape[0] != b.shape[0] or a.shape[2] != b.shape[2]:
        raise ValueError(f"gpa::sim_argmax shape mismatch: a {tuple(a.shape)}, b {tuple(b.shape)}")
    if not _rows_ok(a, 8):
        a = a.contiguous()
    if not _rows_ok(b, 8):
        b = b.contiguous()
    B, M, D = a.shape
    N = b.shape[1]
    max_dtype = a.dtype if max_in_input_dtype else torch.float32
    out_max = torch.empty(B, M, device=dev, dtype=max_dtype)
    out_idx = torch.empty(B, M, device=dev, dtype=torch.int64)
    if B == 0 or M == 0:
        return out_max, out_idx
    L = lib()
    with torch.cuda.device(dev):
        # The plan (and so the workspace size) depends on the current
        # device's CU count: query it with the launch's device current.
        ws_bytes = L.gpa_sim_argmax_workspace_bytes(B, M, N, D)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes else None
        fn = L.gpa_sim_argmax_f16 if a.dtype == torch.float16 else L.gpa_sim_argmax_bf16
        rc = fn(
            a.data_ptr(), b.data_ptr(), out_max.data_ptr(), _DTYPE_CODES[max_dtype],
            out_idx.data_ptr(),
            B, M, N, D, _st(a, 0), _rs(a, 1), _st(b, 0), _rs(b, 1),
            _st(out_max, 0), _st(out_idx, 0),
            ws.data_ptr() if ws is not None else None, ws_bytes, _stream(dev))
    _check(rc, "gpa::sim_argmax")
    return out_max, out_idx


@sim_argmax.register_fake
def _sim_argmax_fake(a, b, max_in_input_dtype=False):
    B, M, _ = a.shape
    return (a.new_empty(B, M, dtype=a.dtype if max_in_input_dtype else torch.float32),
            a.new_empty(B, M, dtype=torch.int64))


# --------------------------------------------------------------------------
# gpa::attn_keybias
# --------------------------------------------------------------------------

# Workspace layout of the attention (gpa_attn_keybias_workspace_bytes): per
# (batch, head) one 144-byte record per 32-key tile, then 16 bytes of row
# bounds per (batch, head), then one flag byte per 64-query wave (4 waves per
# 256-query workgroup).
_ATTN_TILE_KEYS, _ATTN_REC_BYTES, _ATTN_WG_QUERIES, _ATTN_WAVES = 32, 144, 256, 4
_ATTN_BOUND_BYTES = 16
# Bits of a wave's flag: its output comes from the lazily moved offset; it
# took the fixed offset from tile 0 (verified after the loop); its workgroup
# streamed the keys twice (a tile-0 offset of the workgroup overflowed).
ATTN_FLAG_LAZY, ATTN_FLAG_TILE0, ATTN_FLAG_RERUN = 1, 2, 4


def _attn_run(q, k, v, bias, sm_scale, return_lse):
    """Validate, allocate and launch gpa_attn_keybias_{bf16,f16}; returns
    (o, lse, workspace) with the workspace as the kernel left it."""
    tensors = [q, k, v] + ([bias] if bias is not None else [])
    dev = _require_gpu(*tensors)
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"gpa::attn_keybias takes bf16 or fp16 q, got {q.dtype}")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dtype != q.dtype:
            raise ValueError(f"gpa::attn_keybias: {name} is {t.dtype}, q is {q.dtype}")
        if t.dim() != 4:
            raise ValueError(f"gpa::attn_keybias: {name} must be [B,H,T,D], got {tuple(t.shape)}")
    B, H, M, D = q.shape
    N = k.shape[2]
    if k.shape != (B, H, N, D) or v.shape != (B, H, N, D):
        raise ValueError(f"gpa::attn_keybias shape mismatch: q {tuple(q.shape)}, "
                         f"k {tuple(k.shape)}, v {tuple(v.shape)}")
    if not _rows_ok(q, 8):
        q = q.contiguous()
    if not _rows_ok(k, 8):
        k = k.contiguous()
    if not _rows_ok(v, 8):
        v = v.contiguous()
    bias_kind, bias_ptr, bsb, bsh, bsn = GPA_BIAS_NONE, None, 0, 0, 0
    if bias is not None:
        if bias.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            bias = bias.float()
        try:
            bx = bias.expand(B, H, 1, N)
        except RuntimeError as exc:
            raise ValueError(f"gpa::attn_keybias: bias {tuple(bias.shape)} does not broadcast to "
                             f"[B,H,1,N]=[{B},{H},1,{N}]") from exc
        bias_kind = {torch.float32: GPA_BIAS_F32, torch.bfloat16: GPA_BIAS_BF16,
                     torch.float16: GPA_BIAS_F16}[bx.dtype]
        bias_ptr = bx.data_ptr()
        bsb, bsh, bsn = _st(bx, 0), _st(bx, 1), _st(bx, 3)
    o = torch.empty(B, H, M, D, device=dev, dtype=q.dtype)
    lse = (torch.empty(B, H, M, device=dev, dtype=torch.float32) if return_lse
           else torch.empty(0, device=dev, dtype=torch.float32))
    if B == 0 or H == 0 or M == 0:
        return o, lse, None
    L = lib()
    ws_bytes = L.gpa_attn_keybias_workspace_bytes(B, H, M, N)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        fn = L.gpa_attn_keybias_f16 if q.dtype == torch.float16 else L.gpa_attn_keybias_bf16
        rc = fn(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), bias_ptr, bias_kind, bsb, bsh, bsn,
            o.data_ptr(), lse.data_ptr() if return_lse else None,
            B, H, M, N, D,
            _st(q, 0), _st(q, 1), _rs(q, 2),
            _st(k, 0), _st(k, 1), _rs(k, 2),
            _st(v, 0), _st(v, 1), _rs(v, 2),
            _st(o, 0), _st(o, 1), _rs(o, 2),
            _st(lse, 0) if return_lse else 0, _st(lse, 1) if return_lse else 0,
            ws.data_ptr(), ws_bytes, float(sm_scale), _stream(dev))
    _check(rc, "gpa::attn_keybias")
    return o, lse, ws


@torch.library.custom_op("gpa::attn_keybias", mutates_args=())
def attn_keybias(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                 bias: Optional[torch.Tensor], sm_scale: float,
                 return_lse: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """softmax(q k^T * sm_scale + bias) v with a per-key bias.

    q [B,H,M,64], k/v [B,H,N,64], all bf16 or all fp16; bias broadcastable
    to [B,H,1,N] (fp32, bf16 or fp16) or None.  Returns o [B,H,M,64] in q's
    dtype and, if return_lse, the log2 log-sum-exp [B,H,M] fp32 (else an
    empty tensor).
    """
    o, lse, _ = _attn_run(q, k, v, bias, sm_scale, return_lse)
    return o, lse


def attn_keybias_offset_flags(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                              bias: Optional[torch.Tensor], sm_scale: float,
                              return_lse: bool = False):
    """The attention plus which softmax offset each wave used (diagnostic).

    Returns (o, lse, flags) with flags [B*H, ceil(M/256), 4] uint8, one per
    wave of 64 queries: 0 where the score bound certified the fixed offset
    (or the wave holds no query), otherwise the bits ATTN_FLAG_LAZY (the
    output comes from the lazily moved offset), ATTN_FLAG_TILE0 (the wave
    took the fixed offset from tile 0, verified after the loop) and
    ATTN_FLAG_RERUN (a tile-0 offset of its workgroup overflowed, so the
    workgroup streamed the keys again and recomputed with the lazy offset).
    """
    o, lse, ws = _attn_run(q, k, v, bias, sm_scale, return_lse)
    B, H, M, _ = q.shape
    N = k.shape[2]
    if ws is None:
        return o, lse, torch.zeros(0, 0, _ATTN_WAVES, dtype=torch.uint8)
    ntiles = -(-N // _ATTN_TILE_KEYS)
    gx = -(-M // _ATTN_WG_QUERIES)
    start = B * H * ntiles * _ATTN_REC_BYTES + B * H * _ATTN_BOUND_BYTES
    flags = ws[start:start + B * H * gx * _ATTN_WAVES].view(B * H, gx, _ATTN_WAVES)
    return o, lse, flags


@attn_keybias.register_fake
def _attn_keybias_fake(q, k, v, bias, sm_scale, return_lse):
    B, H, M, D = q.shape
    o = q.new_empty(B, H, M, D)
    lse = q.new_empty((B, H, M) if return_lse else (0,), dtype=torch.float32)
    return o, lse


_MERGE_DTYPES = _DTYPE_CODES


@torch.library.custom_op("gpa::merge_heads", mutates_args=())
def merge_heads(t: torch.Tensor, offsets: torch.Tensor, tokens: torch.Tensor, slots: int,
                mean: bool) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Segmented sum / mean of t [B, H, N, D] rows over per-slot token lists.

    offsets [B*slots + 1] and tokens [B*N] (int64, positions within a batch
    element) list every output slot's tokens; returns out [B, H, slots, D]
    in t's dtype, the list lengths [B, slots] and their logs (fp32).
    """
    dev = _require_gpu(t, offsets, tokens)
    if t.dim() != 4:
        raise ValueError(f"gpa::merge_heads: t must be [B,H,N,D], got {tuple(t.shape)}")
    if t.dtype not in _MERGE_DTYPES:
        raise NotImplementedError(f"gpa::merge_heads: dtype {t.dtype} not supported")
    if offsets.dtype != torch.int64 or tokens.dtype != torch.int64:
        raise ValueError("gpa::merge_heads: offsets and tokens must be int64")
    B, H, N, D = t.shape
    if offsets.numel() != B * slots + 1 or tokens.numel() != B * N:
        raise ValueError(f"gpa::merge_heads: offsets {offsets.numel()} / tokens {tokens.numel()} "
                         f"do not match B={B}, slots={slots}, N={N}")
    offsets, tokens = offsets.contiguous(), tokens.contiguous()
    out = torch.empty(B, H, slots, D, device=dev, dtype=t.dtype)
    size = torch.empty(B, slots, device=dev, dtype=torch.float32)
    log_size = torch.empty(B, slots, device=dev, dtype=torch.float32)
    if B == 0 or slots == 0:
        return out, size, log_size
    if not _rows_ok(t, 16 // t.element_size()):
        t = t.contiguous()
    with torch.cuda.device(dev):
        rc = lib().gpa_merge_heads(
            t.data_ptr(), _MERGE_DTYPES[t.dtype], out.data_ptr(),
            offsets.data_ptr(), tokens.data_ptr(), B, H, N, slots, D,
            _st(t, 0), _st(t, 1), _rs(t, 2), _st(out, 0), _st(out, 1), _rs(out, 2),
            GPA_MERGE_MEAN if mean else GPA_MERGE_SUM, size.data_ptr(), log_size.data_ptr(),
            _stream(dev))
    _check(rc, "gpa::merge_heads")
    return out, size, log_size


@merge_heads.register_fake
def _merge_heads_fake(t, offsets, tokens, slots, mean):
    B, H, N, D = t.shape
    return (t.new_empty(B, H, slots, D), t.new_empty(B, slots, dtype=torch.float32),
            t.new_empty(B, slots, dtype=torch.float32))


@torch.library.custom_op("gpa::lse_combine", mutates_args=())
def lse_combine(out_a: torch.Tensor, lse_a: torch.Tensor, out_b: torch.Tensor,
                lse_b: torch.Tensor, frames: int) -> torch.Tensor:
    """Merge the own-frame attention (out_a [B*S, H, P, D], lse_a [B*S, H, P])
    and the shared-set attention (out_b [B, H, S*P, D], lse_b [B, H, S*P]) by
    their log2 LSE; returns y [B, S*P, H*D] in the outputs' dtype (bf16 or
    fp16, the same for both)."""
    dev = _require_gpu(out_a, lse_a, out_b, lse_b)
    for name, t in (("out_a", out_a), ("out_b", out_b)):
        if t.dtype not in (torch.bfloat16, torch.float16) or t.dtype != out_a.dtype \
                or t.dim() != 4:
            raise ValueError(f"gpa::lse_combine: {name} must be bf16 or fp16 (both alike) "
                             f"[.,H,.,D], got {t.dtype} {tuple(t.shape)}")
    for name, t in (("lse_a", lse_a), ("lse_b", lse_b)):
        if t.dtype != torch.float32 or t.dim() != 3:
            raise ValueError(f"gpa::lse_combine: {name} must be fp32 [.,H,.], got "
                             f"{t.dtype} {tuple(t.shape)}")
    S = int(frames)
    BS, H, P, D = out_a.shape
    B, Hb, N, Db = out_b.shape
    if S <= 0 or BS != B * S or Hb != H or Db != D or N != S * P or \
            tuple(lse_a.shape) != (BS, H, P) or tuple(lse_b.shape) != (B, H, N):
        raise ValueError(f"gpa::lse_combine: shapes do not match: out_a {tuple(out_a.shape)}, "
                         f"lse_a {tuple(lse_a.shape)}, out_b {tuple(out_b.shape)}, "
                         f"lse_b {tuple(lse_b.shape)}, frames {frames}")
    if not _rows_ok(out_a, 8):
        out_a = out_a.contiguous()
    if not _rows_ok(out_b, 8):
        out_b = out_b.contiguous()
    y = torch.empty(B, N, H * D, device=dev, dtype=out_a.dtype)
    if y.numel() == 0:
        return y
    sa0, sa1, sa2 = out_a.stride()[:3]
    la0, la1, la2 = lse_a.stride()
    sb0, sb1, sb2 = out_b.stride()[:3]
    lb0, lb1, lb2 = lse_b.stride()
    with torch.cuda.device(dev):
        fn = lib().gpa_lse_combine_f16 if out_a.dtype == torch.float16 \
            else lib().gpa_lse_combine_bf16
        rc = fn(
            out_a.data_ptr(), lse_a.data_ptr(), out_b.data_ptr(), lse_b.data_ptr(), y.data_ptr(),
            B, H, N, P, D,
            S * sa0, sa1, sa0, sa2,            # out_a (b, h, s, p)
            S * la0, la1, la0, la2,            # lse_a
            sb0, sb1, P * sb2, sb2,            # out_b (b, h, s, p), token n = s*P + p
            lb0, lb1, P * lb2, lb2,            # lse_b
            y.stride(0), y.stride(1), D,       # y (b, n, h)
            _stream(dev))
    _check(rc, "gpa::lse_combine")
    return y


@lse_combine.register_fake
def _lse_combine_fake(out_a, lse_a, out_b, lse_b, frames):
    B, H, N, D = out_b.shape
    return out_b.new_empty(B, N, H * D, dtype=out_a.dtype)


@torch.library.custom_op("gpa::qk_norm_rope", mutates_args=())
def qk_norm_rope(qkv: torch.Tensor, ln_w: torch.Tensor, ln_b: torch.Tensor, eps: float,
                 pos: Optional[torch.Tensor], rope_cs: Optional[torch.Tensor], heads: int,
                 q_f32: bool, k_f32: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """qk LayerNorm + 2D RoPE of the QKV projection qkv [B, N, >= 3*heads*64]
    (bf16 or fp16): returns q, k [B, heads, N, 64], each fp32 or of qkv's
    16-bit format.

    ln_w / ln_b [2, 64]: the q and k LayerNorm affine parameters; pos
    [period, 2] int32 (token n uses row n mod period) and rope_cs
    [npos, 16, 2] fp32 (cos, sin) tables, or both None for no rotation.
    """
    dev = _require_gpu(qkv, ln_w, ln_b)
    if qkv.dtype not in (torch.bfloat16, torch.float16) or qkv.dim() != 3:
        raise ValueError(f"gpa::qk_norm_rope: qkv must be bf16 or fp16 [B, N, 3C], got "
                         f"{qkv.dtype} {tuple(qkv.shape)}")
    H = int(heads)
    if H <= 0 or qkv.shape[2] < 3 * H * 64:
        raise ValueError(f"gpa::qk_norm_rope: rows of {qkv.shape[2]} cannot hold q, k, v of "
                         f"{H} heads x 64")
    w = ln_w.to(device=dev, dtype=torch.float32).contiguous()
    bb = ln_b.to(device=dev, dtype=torch.float32).contiguous()
    if w.numel() != 128 or bb.numel() != 128:
        raise ValueError("gpa::qk_norm_rope: ln_w and ln_b hold the q and k weights, 2 x 64")
    if (pos is None) != (rope_cs is None):
        raise ValueError("gpa::qk_norm_rope: pos and rope_cs go together")
    period, npos = 0, 0
    if pos is not None:
        _require_gpu(pos, rope_cs)
        if pos.dtype != torch.int32 or pos.dim() != 2 or pos.shape[1] != 2:
            raise ValueError("gpa::qk_norm_rope: pos must be int32 [period, 2]")
        if rope_cs.dtype != torch.float32 or rope_cs.shape[1:] != (16, 2):
            raise ValueError("gpa::qk_norm_rope: rope_cs must be fp32 [npos, 16, 2]")
        pos, rope_cs = pos.contiguous(), rope_cs.contiguous()
        period, npos = pos.shape[0], rope_cs.shape[0]
    if not _rows_ok(qkv, 8):
        qkv = qkv.contiguous()
    B, N, _ = qkv.shape
    f16 = qkv.dtype == torch.float16
    half, half_code = (torch.float16, GPA_DTYPE_F16) if f16 else (torch.bfloat16, GPA_DTYPE_BF16)
    q = torch.empty(B, H, N, 64, device=dev, dtype=torch.float32 if q_f32 else half)
    k = torch.empty(B, H, N, 64, device=dev, dtype=torch.float32 if k_f32 else half)
    if q.numel() == 0:
        return q, k
    with torch.cuda.device(dev):
        fn = lib().gpa_qk_norm_rope_f16 if f16 else lib().gpa_qk_norm_rope_bf16
        rc = fn(
            qkv.data_ptr(), B, N, H, 64, _st(qkv, 0), _rs(qkv, 1), H * 64,
            w.data_ptr(), bb.data_ptr(), float(eps),
            pos.data_ptr() if pos is not None else None, period,
            rope_cs.data_ptr() if rope_cs is not None else None, npos,
            q.data_ptr(), GPA_DTYPE_F32 if q_f32 else half_code,
            k.data_ptr(), GPA_DTYPE_F32 if k_f32 else half_code, _stream(dev))
    _check(rc, "gpa::qk_norm_rope")
    return q, k


@qk_norm_rope.register_fake
def _qk_norm_rope_fake(qkv, ln_w, ln_b, eps, pos, rope_cs, heads, q_f32, k_f32):
    B, N, _ = qkv.shape
    half = qkv.dtype if qkv.dtype in (torch.bfloat16, torch.float16) else torch.bfloat16
    return (qkv.new_empty(B, heads, N, 64, dtype=torch.float32 if q_f32 else half),
            qkv.new_empty(B, heads, N, 64, dtype=torch.float32 if k_f32 else half))


@torch.library.custom_op("gpa::pool_shared", mutates_args=())
def pool_shared(k: torch.Tensor, v: torch.Tensor, frames: int, pts: int, grid_h: int,
                grid_w: int, kp: int, want_assign: bool
                ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Pooled summaries of the frame-special shared set from k, v [B, H, S*P, 64]
    (both bf16 or both fp16) on a grid_h x grid_w patch grid: returns pooled
    k, v [B, H, S*npool, 64] in that format, size [B, H, S, npool] fp32 and, if asked, the
    assignment [B, H, S, grid_h*grid_w] int32 (else empty);
    npool = ceil(grid_h/kp) * ceil(grid_w/kp)."""
    dev = _require_gpu(k, v)
    for name, t in (("k", k), ("v", v)):
        if t.dtype not in (torch.bfloat16, torch.float16) or t.dim() != 4 or t.dtype != k.dtype:
            raise ValueError(f"gpa::pool_shared: {name} must be bf16 or fp16 [B,H,N,64] like k, "
                             f"got {t.dtype} {tuple(t.shape)}")
    if k.shape != v.shape:
        raise ValueError(f"gpa::pool_shared: k {tuple(k.shape)} and v {tuple(v.shape)} differ")
    if kp <= 0 or grid_h < 0 or grid_w < 0:
        raise ValueError(f"gpa::pool_shared: grid {grid_h}x{grid_w}, kp {kp}")
    B, H, N, D = k.shape
    S = int(frames)
    if S <= 0 or N % S != 0:
        raise ValueError(f"gpa::pool_shared: {N} tokens do not split into {S} frames")
    P = N // S
    npool = -(-int(grid_h) // int(kp)) * -(-int(grid_w) // int(kp))
    if not _rows_ok(k, 8):
        k = k.contiguous()
    if not _rows_ok(v, 8):
        v = v.contiguous()
    pk = torch.empty(B, H, S * npool, D, device=dev, dtype=k.dtype)
    pv = torch.empty(B, H, S * npool, D, device=dev, dtype=k.dtype)
    size = torch.empty(B, H, S, npool, device=dev, dtype=torch.float32)
    assign = (torch.empty(B, H, S, grid_h * grid_w, device=dev, dtype=torch.int32)
              if want_assign else torch.empty(0, device=dev, dtype=torch.int32))
    if pk.numel() == 0:
        return pk, pv, size, assign
    with torch.cuda.device(dev):
        fn = lib().gpa_pool_shared_f16 if k.dtype == torch.float16 else lib().gpa_pool_shared_bf16
        rc = fn(
            k.data_ptr(), v.data_ptr(), pk.data_ptr(), pv.data_ptr(), size.data_ptr(),
            assign.data_ptr() if want_assign else None, B, H, S, P, pts, grid_h, grid_w, kp, D,
            _st(k, 0), _st(k, 1), _rs(k, 2), _st(v, 0), _st(v, 1), _rs(v, 2), _stream(dev))
    _check(rc, "gpa::pool_shared")
    return pk, pv, size, assign


@pool_shared.register_fake
def _pool_shared_fake(k, v, frames, pts, grid_h, grid_w, kp, want_assign):
    B, H, N, D = k.shape
    npool = -(-grid_h // kp) * -(-grid_w // kp)
    return (k.new_empty(B, H, frames * npool, D), k.new_empty(B, H, frames * npool, D),
            k.new_empty(B, H, frames, npool, dtype=torch.float32),
            k.new_empty((B, H, frames, grid_h * grid_w) if want_assign else (0,),
                        dtype=torch.int32))


# --------------------------------------------------------------------------
# gpa::merge_metric
# --------------------------------------------------------------------------

_METRIC_DTYPES = {torch.float32: GPA_DTYPE_F32, torch.bfloat16: GPA_DTYPE_BF16}


@torch.library.custom_op("gpa::merge_metric", mutates_args=())
def merge_metric(metric: torch.Tensor, proj: torch.Tensor, order: Optional[torch.Tensor],
                 mode: int) -> torch.Tensor:
    """bf16(normalise(round(round(metric[:, order]) @ proj))) as [B, N, 128] bf16.

    metric [B, N, C] fp32 or bf16 (C in 256, 512, 768, 1024), order [N] int64
    token positions (None: identity).  mode 0: bf16 projection (proj [C, 128]
    bf16), fp32 norm -- the chain under bf16 autocast; 1: the same with the
    norm rounded to bf16 -- a bf16 metric without autocast; 2: fp16 projection
    (proj fp16, fp32 metric), fp32 norm -- the chain under fp16 autocast."""
    dev = _require_gpu(metric, proj)
    if metric.dim() != 3 or metric.dtype not in _METRIC_DTYPES:
        raise ValueError(f"gpa::merge_metric: metric must be fp32/bf16 [B,N,C], got "
                         f"{metric.dtype} {tuple(metric.shape)}")
    if mode not in (0, 1, 2):
        raise ValueError(f"gpa::merge_metric: mode {mode} is not 0, 1 or 2")
    B, N, C = metric.shape
    want = torch.float16 if mode == 2 else torch.bfloat16
    if proj.dtype != want or proj.dim() != 2 or proj.shape[0] != C:
        raise ValueError(f"gpa::merge_metric: mode {mode} takes a {want} proj [{C}, P], got "
                         f"{proj.dtype} {tuple(proj.shape)}")
    P = proj.shape[1]
    proj = proj.contiguous()
    if order is not None:
        _require_gpu(order)
        if order.dtype != torch.int64 or order.shape != (N,):
            raise ValueError(f"gpa::merge_metric: order must be int64 [{N}], got {order.dtype} "
                             f"{tuple(order.shape)}")
        order = order.contiguous()
    if not _rows_ok(metric, 16 // metric.element_size()):
        metric = metric.contiguous()
    out = torch.empty(B, N, P, device=dev, dtype=torch.bfloat16)
    if out.numel() == 0:
        return out
    with torch.cuda.device(dev):
        rc = lib().gpa_merge_metric_bf16(
            metric.data_ptr(), _METRIC_DTYPES[metric.dtype], B, N, C, _st(metric, 0),
            _rs(metric, 1), proj.data_ptr(), P, None if order is None else order.data_ptr(),
            int(mode), out.data_ptr(), _stream(dev))
    _check(rc, "gpa::merge_metric")
    return out


@merge_metric.register_fake
def _merge_metric_fake(metric, proj, order, mode):
    B, N, _ = metric.shape
    return metric.new_empty(B, N, proj.shape[1], dtype=torch.bfloat16)


# --------------------------------------------------------------------------
# gpa::residual_layernorm
# --------------------------------------------------------------------------

@torch.library.custom_op("gpa::residual_layernorm", mutates_args=())
def residual_layernorm(x: torch.Tensor, y: Optional[torch.Tensor], gamma: Optional[torch.Tensor],
                       weight: Optional[torch.Tensor], bias: Optional[torch.Tensor], eps: float,
                       want_h: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """h = r(x + r(gamma * y)) (h = x without y) and LayerNorm(h), rounded
    (r) to x's 16-bit format, over the last dim of x / y; all tensors bf16, or
    all fp16.  Returns (h if want_h else an empty tensor, LayerNorm(h) if
    weight is given else an empty tensor)."""
    dev = _require_gpu(*[t for t in (x, y, gamma, weight, bias) if t is not None])
    C = x.shape[-1]
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"gpa::residual_layernorm takes bf16 or fp16 x, got {x.dtype}")
    for name, t in (("y", y), ("gamma", gamma), ("weight", weight), ("bias", bias)):
        if t is not None and t.dtype != x.dtype:
            raise ValueError(f"gpa::residual_layernorm: {name} is {t.dtype}, x is {x.dtype}")
    if y is not None and (y.shape != x.shape or gamma is None or gamma.shape != (C,)):
        raise ValueError("gpa::residual_layernorm: y must match x and gamma be [C]")
    if weight is not None and (bias is None or weight.shape != (C,) or bias.shape != (C,)):
        raise ValueError("gpa::residual_layernorm: weight and bias must be [C]")
    if want_h and y is None:
        raise ValueError("gpa::residual_layernorm: want_h needs y")
    xr = x.reshape(-1, C)
    if not _rows_ok(xr, 8):
        xr = xr.contiguous()
    yr = None
    if y is not None:
        yr = y.reshape(-1, C)
        if not _rows_ok(yr, 8):
            yr = yr.contiguous()
        gamma = gamma.contiguous()
    if weight is not None:
        weight, bias = weight.contiguous(), bias.contiguous()
    rows = xr.shape[0]
    h = torch.empty(x.shape, device=dev, dtype=x.dtype) if want_h else x.new_empty(0)
    ln = torch.empty(x.shape, device=dev, dtype=x.dtype) if weight is not None \
        else x.new_empty(0)
    if rows == 0:
        return h, ln
    with torch.cuda.device(dev):
        fn = (lib().gpa_residual_layernorm_f16 if x.dtype == torch.float16
              else lib().gpa_residual_layernorm_bf16)
        rc = fn(
            xr.data_ptr(), None if yr is None else yr.data_ptr(),
            None if gamma is None else gamma.data_ptr(),
            None if weight is None else weight.data_ptr(),
            None if bias is None else bias.data_ptr(), float(eps), rows, C,
            _rs(xr, 0), 0 if yr is None else _rs(yr, 0),
            h.data_ptr() if want_h else None, C, ln.data_ptr() if weight is not None else None, C,
            _stream(dev))
    _check(rc, "gpa::residual_layernorm")
    return h, ln


@residual_layernorm.register_fake
def _residual_layernorm_fake(x, y, gamma, weight, bias, eps, want_h):
    return (x.new_empty(x.shape if want_h else (0,)),
            x.new_empty(x.shape if weight is not None else (0,)))
