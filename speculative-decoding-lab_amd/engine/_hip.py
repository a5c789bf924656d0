"""ctypes binding of libspecverify.so (the gfx950 HIP library).

There is no CPU path: every operation of this package runs on the GPU through
this library, and loading fails loudly when the library has not been built or a
tensor is not on a GPU device.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "lib", "libspecverify.so")

SPV_OK = 0
SPV_ERR_ARG = -1
SPV_ERR_LAUNCH = -2
SPV_ERR_WORKSPACE = -3
SPV_ERR_UNSUPPORTED = -4
SPV_CTR_WORDS = 16
CTR_TOP, CTR_EXHAUSTED, CTR_SLOWPATH, CTR_PUSHED = 0, 1, 2, 3
CTR_OVERFLOW, CTR_BAD_READ, CTR_ALIGN = 6, 7, 8  # sticky error words (see include/specverify.h)
# bits of a sequence's flag word (sampling): a result the reference may have decided otherwise
FLAG_ACCEPT_BAND, FLAG_DRAW_BAND, FLAG_TOP_P_BAND = 1, 2, 4

SPV_F32, SPV_BF16, SPV_F16, SPV_FP8E4M3 = 0, 1, 2, 3
_DTYPE_CODE = {torch.float32: SPV_F32, torch.bfloat16: SPV_BF16, torch.float16: SPV_F16}
if hasattr(torch, "float8_e4m3fn"):
    _DTYPE_CODE[torch.float8_e4m3fn] = SPV_FP8E4M3

_ERRORS = {
    SPV_ERR_ARG: "invalid argument",
    SPV_ERR_LAUNCH: "kernel launch failed",
    SPV_ERR_WORKSPACE: "workspace too small",
    SPV_ERR_UNSUPPORTED: "unsupported configuration",
}

P = ctypes.c_void_p
I = ctypes.c_int32
F = ctypes.c_float
S = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/specverify.h
SIGNATURES = {
    "spv_version": (ctypes.c_char_p, []),
    "spv_pool_init": (I, [P, P, P, I, P]),
    "spv_pool_alloc_one": (I, [P, P, P, I, P, P]),
    "spv_pool_free_one": (I, [P, P, P, I, I, P, P]),
    "spv_kv_append": (I, [P, P, I, P, P, P, I, P, P, P, P, P, P, P, I, I, I, I, I, I, I, I, I, P]),
    "spv_kv_append_plan": (I, [P, P, I, P, P, P, I, P, P, P, P, P, P, P, I, I, I, I, I, I, I, I, I, P, P]),
    "spv_kv_write_planned": (I, [P, P, I, P, P, P, I, I, I, I, I, I, I, P]),
    "spv_kv_append_fp8": (I, [P, P, P, I, P, P, P, I, P, P, P, P, P, P, P, I, I, I, I, I, I, I, I, I, I, P]),
    "spv_kv_rewind": (I, [P, I, P, P, P, P, P, P, P, P, I, I, I, I, P]),
    "spv_kv_rewind_append": (I, [P, P, I, P, P, P, I, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, P, P]),
    "spv_kv_draft_align": (I, [P, I, P, P, P, P, P, P, I, P, P, P, P, P, I, P, P, P, I, I, I, P]),
    "spv_pool_metrics": (I, [P, P, I, I, P, P, I, P, P, P]),
    "spv_kv_gather": (I, [P, P, I, P, P, I, I, I, I, I, I, I, I, P, P]),
    "spv_kv_read_blocks": (I, [P, I, I, P, I, I, I, I, I, I, P, P]),
    "spv_verify_attn_workspace_bytes": (S, [I, I, I, I, I, I, I]),
    "spv_verify_attn": (I, [P, P, I, P, P, I, P, P, I, P, P, P, P, I, I, I, I, I, I, I, I, I, F, P, S, P]),
    "spv_verify_attn_plan_bytes": (S, [I]),
    "spv_verify_attn_plan": (I, [P, I, P, P, P, P, I, I, I, I, I, I, I, I, I, P, S, P]),
    "spv_verify_attn_planned": (I, [P, P, I, P, P, I, P, P, I, P, P, P, P, I, I, I, I, I, I, I, I, I, F, P, P, S, P]),
    "spv_prefill_attn": (I, [P, P, P, P, I, P, I, I, I, I, I, F, P]),
    "spv_time_next_attention": (I, [P, P]),
    "spv_verify_attn_static_max_bytes": (S, []),
    "spv_verify_attn_static": (I, [P, P, I, P, P, I, P, P, I, P, P, P, P, I, I, I, I, I, I, I, I, I, F, P]),
    "spv_verify_sample_workspace_bytes": (S, [I, I, I]),
    "spv_verify_sample": (I, [P, P, I, F, P, P, P, P, P, P, I, I, I, I, P, P, P, P, P, P, P, I, P, S, P]),
    "spv_draft_sample_workspace_bytes": (S, [I, I]),
    "spv_draft_sample": (I, [P, ctypes.c_int64, F, P, I, I, P, I, P, P, P, S, P]),
    "spv_filter_logits": (I, [P, ctypes.c_int64, P, ctypes.c_int64, I, I, F, I, F, P, P]),
    "spv_logits_to_probs": (I, [P, P, I, I, F, P]),
    "spv_residual": (I, [P, P, P, I, P]),
    "spv_race_argmax": (I, [P, P, I, P, P]),
    "spv_accept_prob": (I, [P, P, I, P, P]),
}


class HipLibraryError(RuntimeError):
    """The HIP library is missing or a call into it failed."""


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load libspecverify.so once (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipLibraryError(
                "libspecverify.so not found at {}; build it with "
                "`python speculative-decoding-lab_amd/build.py`".format(LIB_PATH))
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


_fns: dict = {}


def call(name: str, *args) -> None:
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(lib(), name)
    rc = fn(*args)
    if rc != SPV_OK:
        raise HipLibraryError("{} failed: {} ({})".format(name, _ERRORS.get(rc, "error"), rc))


def require_gpu(device: torch.device) -> torch.device:
    device = torch.device(device)
    if device.type != "cuda":
        raise HipLibraryError(
            "this engine runs on the GPU only (got device {!r}); there is no CPU path".format(str(device)))
    if not torch.cuda.is_available():
        raise HipLibraryError("no GPU is visible to PyTorch")
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    return device


def stream_of(device: torch.device) -> int:
    """The raw handle of ``device``'s current stream (the capturing stream
    inside a graph capture)."""
    idx = device.index if isinstance(device, torch.device) else torch.device(device).index
    if idx is None:
        idx = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


def dtype_code(dtype: torch.dtype) -> int:
    if dtype not in _DTYPE_CODE:
        raise HipLibraryError("unsupported dtype {}".format(dtype))
    return _DTYPE_CODE[dtype]


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def filtering(top_k: int, top_p: float, vocab: int) -> bool:
    """Whether top-k / top-p change a row of ``vocab`` logits."""
    return (0 < int(top_k) < int(vocab)) or (0.0 < float(top_p) < 1.0)


def filter_rows(z: torch.Tensor, temperature: float, top_k: int, top_p: float, ambiguous: bool = False):
    """``spv_filter_logits`` over the rows of a float32 (..., V) tensor: the
    scaled logits with what top-k / top-p drop set to -inf (a new tensor).
    With ``ambiguous``, also the int32 count per row (shape ``z.shape[:-1]``)
    of values whose preceding mass lies within the rounding window of the
    nucleus edge, where the reference's fp32 softmax may keep or drop them
    otherwise: returns ``(out, counts)``."""
    z = z.float().contiguous()
    V = int(z.shape[-1])
    rows = z.numel() // V if V else 0
    out = torch.empty_like(z)
    amb = torch.empty(z.shape[:-1], dtype=torch.int32, device=z.device) if ambiguous else None
    call("spv_filter_logits", ptr(z), V, ptr(out), V, rows, V, float(temperature), int(top_k), float(top_p),
         ptr(amb), stream_of(z.device))
    return (out, amb) if ambiguous else out


def i32(values, device: torch.device) -> torch.Tensor:
    """int32 device tensor from a tensor or a Python sequence."""
    if isinstance(values, torch.Tensor):
        return values.to(device=device, dtype=torch.int32).contiguous()
    return torch.tensor(list(values), dtype=torch.int32, device=device)


class Workspace:
    """Device scratch of one family of entry points, owned by the caller of the
    library: one zero-filled, grow-only buffer per (device, stream).

    The attention and sampling entry points keep arrival counters at its head
    that must start at zero (and are zero again after every call), and calls
    that share a buffer must be ordered: giving each stream its own buffer
    keeps calls on two streams from racing on counters and partials. A buffer
    replaced by a larger one is kept alive for the life of the object, since a
    HIP graph captured earlier may still point at it."""

    def __init__(self) -> None:
        self._bufs: dict = {}
        self._retired: list = []

    @staticmethod
    def _key(device: torch.device, stream: Optional[int] = None):
        device = torch.device(device)
        return device.index, stream_of(device) if stream is None else stream

    def get(self, nbytes: int, device: torch.device, stream: Optional[int] = None) -> torch.Tensor:
        """The buffer of ``stream`` (default: the current stream) on ``device``."""
        key = self._key(device, stream)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                self._retired.append(buf)
            buf = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf

    def current(self, device: torch.device) -> Optional[torch.Tensor]:
        """The buffer of the current stream on ``device`` (None before first use)."""
        return self._bufs.get(self._key(device))
