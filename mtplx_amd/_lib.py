"""ctypes binding of ``libmtplx_amd.so`` (the C ABI in ``include/mtplx_amd.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime
torch already mapped (one runtime per process). There is no CPU fallback: if
the library is missing or a call fails, :class:`MtpError` is raised.
"""

from __future__ import annotations

import ctypes as C
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmtplx_amd.so")

_vp = C.c_void_p
_i = C.c_int
_f = C.c_float
_d = C.c_double
_sz = C.c_size_t

# name -> (restype, argtypes); mirrors include/mtplx_amd.h.
SIGNATURES = {
    "mtp_last_error": (C.c_char_p, []),
    "mtp_qmv_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "mtp_qmv_rope_fusable": (_i, [_i, _i, _i]),
    "mtp_qmv_affine4": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "mtp_qmv_affine": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "mtp_chunk_sums": (_i, [_vp, _i, _i, _vp, _vp]),
    "mtp_crossrow_qmm": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "mtp_qmv_affine4_residual": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "mtp_qmv_affine4_dual": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "mtp_qmv_affine4_swiglu_in": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "mtp_qmv_affine4_rmsnorm_in": (_i, [_vp, _vp, _vp, _f, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "mtp_qmv_affine4_rmsnorm_f32": (_i, [_vp, _vp, _vp, _f, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "mtp_qmv_affine4_rmsnorm_dual": (_i, [_vp, _vp, _vp, _f, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i,
                                          _vp, _sz, _vp]),
    "mtp_kv_scatter": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp]),
    "mtp_kv_restore_masked": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "mtp_ragged_causal_mask": (_i, [_vp, _vp, _i, _i, _i, _vp]),
    "mtp_attn_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "mtp_ragged_gqa_attn": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _i, _vp, _sz, _vp]),
    "mtp_ragged_gqa_attn_rows": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _i, _vp, _sz,
                                      _vp]),
    "mtp_rope_qkv_to_cache": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _vp, _vp]),
    "mtp_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _f, _vp]),
    "mtp_embed_affine4": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp]),
    "mtp_sampler_workspace_bytes": (_sz, [_i, _i, _i]),
    "mtp_spec_accept": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _d, _i, _d, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mtp_spec_accept_ragged": (_i, [_vp, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _d, _i, _d, _vp, _vp, _vp,
                                    _vp, _vp, _sz, _vp]),
    "mtp_spec_accept_noalloc": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _d, _i, _d, _vp, _vp, _vp, _vp, _vp]),
    "mtp_sample_rows": (_i, [_vp, _i, _i, _d, _i, _d, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mtp_apply_logit_deltas": (_i, [_vp, C.c_longlong, _i, _i, _vp, _vp, _vp, _i, _vp, _vp]),
    "mtp_probe_mfma_layout": (_i, [_vp, _vp]),
    "mtp_moe_workspace_bytes": (_sz, [_i, _i, _i]),
    "mtp_moe_sort": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mtp_gather_qmv_affine4": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i,
                                    _i, _i, _i, _i, _vp, _sz, _vp]),
    "mtp_gather_qmv_affine4_packed": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "mtp_gather_qmv_affine4_packed_rows": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "mtp_gather_qmv_affine4_packed_mf16": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "mtp_moe_route": (_i, [_vp, _i, _vp, _i, _i, _i, _vp, _vp, _vp]),
    "mtp_moe_segments": (_i, [_vp, _i, _i, _vp, _vp, _vp]),
    "mtp_moe_combine": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _vp]),
    "mtp_moe_combine_ss": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "mtp_pack_affine4_bytes": (_sz, [_i, _i]),
    "mtp_pack_affine4": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "mtp_pack_affine4_mf16": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "mtp_qmv_affine4_ex": (_i, [_vp, _vp]),
    "mtp_qmm_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "mtp_qmm_affine4_mfma": (_i, [_vp, _vp]),
    "mtp_attn_blocks_workspace_bytes": (_sz, [_i, _i, _i, C.c_longlong, _i]),
    "mtp_ragged_gqa_attn_blocks": (_i, [_vp, _vp]),
    "mtp_rope_qkv_to_blocks": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _vp, _vp]),
    "mtp_attn_vt_workspace_bytes": (_sz, [_i, _i, _i]),
    "mtp_ragged_gqa_attn_rows_vt": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _vp, _sz, _vp]),
    "mtp_rope_qkv_to_cache_vt": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _vp, _vp]),
}


class RopeOut(C.Structure):
    """``mtp_rope_out`` of include/mtplx_amd.h (same field order)."""

    _fields_ = [(n, _vp) for n in ("q_start", "q_lens", "q_out", "k_cache", "v_cache", "status")] + \
               [(n, _i) for n in ("L", "Hq", "Hkv", "D", "cap", "blocked")] + [("rope_base", _f)]


class QmvArgs(C.Structure):
    """``mtp_qmv_args`` of include/mtplx_amd.h (same field order)."""

    _fields_ = [(n, _vp) for n in ("x", "x2", "ss_in", "w0", "s0", "b0", "w1", "s1", "b1", "y0", "y1", "yf",
                                   "resid", "ss_out")] + [("eps", _f)] + \
               [(n, _i) for n in ("M", "N", "K", "group_size", "ldx", "ldy", "xmode", "emode", "packed")] + \
               [("ws", _vp), ("ws_bytes", C.c_size_t), ("rope", C.POINTER(RopeOut)), ("schedule", _i)] + \
               [(n, _vp) for n in ("x_sums", "y_sums")]


def _fill(struct, fields: dict):
    for k, v in fields.items():
        if hasattr(v, "data_ptr"):
            v = v.data_ptr()
        setattr(struct, k, v)
    return struct


def qmv_ex(stream, rope: dict | None = None, **fields) -> None:
    """Call ``mtp_qmv_affine4_ex``; tensor fields may be torch tensors or None.
    ``rope``: fields of ``mtp_rope_out`` (emode 4)."""
    a = _fill(QmvArgs(), fields)
    r = None
    if rope is not None:
        r = _fill(RopeOut(), rope)
        a.rope = C.pointer(r)
    call("mtp_qmv_affine4_ex", C.byref(a), stream)


class QmmArgs(C.Structure):
    """``mtp_qmm_args`` of include/mtplx_amd.h (same field order)."""

    _fields_ = [(n, _vp) for n in ("x", "w0", "w1", "y", "yf", "resid")] + \
               [(n, _i) for n in ("M", "N", "K", "group_size", "ldx", "ldy", "emode")] + \
               [("ws", _vp), ("ws_bytes", C.c_size_t)]


def qmm_mfma(stream, **fields) -> None:
    """Call ``mtp_qmm_affine4_mfma``; tensor fields may be torch tensors or None."""
    call("mtp_qmm_affine4_mfma", C.byref(_fill(QmmArgs(), fields)), stream)


class AttnBlocksArgs(C.Structure):
    """``mtp_attn_blocks_args`` of include/mtplx_amd.h (same field order)."""

    _fields_ = [(n, _vp) for n in ("q", "k_blk", "v_blk", "q_start", "q_lens", "row_off", "kv_off", "out")] + \
               [(n, _i) for n in ("B", "Hq", "Hkv", "Lmax", "D", "cap", "split_keys")] + \
               [("scale", _f), ("total_cap", C.c_longlong), ("ws", _vp), ("ws_bytes", C.c_size_t)]


def attn_blocks(stream, **fields) -> None:
    """Call ``mtp_ragged_gqa_attn_blocks``; tensor fields may be torch tensors or None."""
    call("mtp_ragged_gqa_attn_blocks", C.byref(_fill(AttnBlocksArgs(), fields)), stream)


class MtpError(RuntimeError):
    """A C-ABI call failed (message from ``mtp_last_error``)."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


_LIB = None
_LOCK = threading.Lock()


def load():
    """Load the library once (after torch) and bind every declared symbol."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        import torch  # noqa: F401  -- bind to the HIP runtime torch mapped

        if not os.path.exists(LIB_PATH):
            raise MtpError("load", -4, f"{LIB_PATH} is missing; run `python -m mtplx_amd.build`")
        lib = C.CDLL(LIB_PATH, mode=C.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
        return lib


def call(name: str, *args) -> int:
    """Call ``name`` and raise :class:`MtpError` on a non-zero return."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.mtp_last_error().decode(errors="replace")
        raise MtpError(name, rc, msg)
    return rc


def query(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))


# ---------------------------------------------------------------------------
# torch plumbing: pointers, streams, workspaces.

def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device=None) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream


class _Workspaces:
    """One zero-initialised byte buffer per (device, stream, tag), grown on demand.

    Kernels keep self-resetting arrival counters in their workspace, so a
    buffer is zero-filled only when it is (re)allocated.
    """

    def __init__(self):
        self._bufs: dict = {}

    def get(self, nbytes: int, tag: str, device=None):
        import torch

        idx = None if device is None else torch.device(device).index
        dev = torch.device("cuda", torch.cuda.current_device() if idx is None else idx)   # "cuda" = current device
        key = (dev.index, stream_handle(dev), tag)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            size = max(int(nbytes), 256)
            if buf is not None:
                size = max(size, 2 * buf.numel())
            buf = torch.zeros(size, dtype=torch.uint8, device=dev)
            self._bufs[key] = buf
        return buf


WORKSPACES = _Workspaces()
