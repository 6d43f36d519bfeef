"""ctypes binding of libsemblend_hip.so (the C ABI declared in include/semblend_hip.h).

The library is loaded after ``import torch`` so that it binds to the HIP runtime torch already
loaded (both carry the ``libamdhip64.so.7`` soname); device pointers and hipStream_t handles
from torch are then valid in the library. There is no fallback: if the library is missing or
fails to load, every kernel entry point raises ``RuntimeError``.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
from pathlib import Path

import torch

# The library built in-tree next to this file (semblend_amd/_build.py writes it).
LIB_PATH = Path(__file__).resolve().parent / "libsemblend_hip.so"

SB_OK = 0
SB_ERR_INVALID_ARGUMENT = 100001
# Flag of the multi-layer scatters: a donor row may be the source of several pairs.
SB_SCATTER_REPEATED_DONOR_ROWS = 1
# Most positions the in-place delta RoPE takes by value in its launch (host arrays).
SB_INLINE_POSITIONS_MAX = 256
# Segment alignment (pairs) of the donor-grouped composite scatter.
SB_GROUPED_PAIR_ALIGN = 256
# Constant RoPE deltas must lie strictly within +-2^31 (the C ABI's check; the kernels'
# sin/cos reduce angles below 2^32 exactly).
MAX_ROPE_DELTA = 1 << 31
SB_DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)
I32P = _i32p  # host int32 arrays passed by address (numpy: arr.ctypes.data_as(I32P))

# Argument signatures of every exported function (order as in include/semblend_hip.h).
SIGNATURES: dict[str, list] = {
    "sb_scatter_donor_kv": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64p,
                            _i64p, _i32, _vp],
    "sb_scatter_donor_kv_paged": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                  _i64, _i64p, _i64p, _i32, _vp],
    "sb_scatter_donor_kv_paged_layers": [_vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                         _i64, _i64, _i64, _i64p, _i64p, _i32, _i32, _vp],
    "sb_rope_correct_scatter_paged": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                      _i64, _i64, _i64, _i64p, _i64p, _i32, _vp],
    "sb_rope_correct_scatter_paged_layers": [_vp, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64,
                                             _i64, _i64, _i64, _i64, _i64, _i64p, _i64p, _i32,
                                             _i32, _vp],
    "sb_composite_scatter_paged_layers": [_vp, _i64, _vp, _i64, _i64p, _vp, _vp, _vp, _vp,
                                          _i64, _i64, _i64, _i64, _vp, _i64, _i64, _i64p, _i32,
                                          _i32, _vp],
    "sb_composite_scatter_paged_layers_grouped": [_vp, _i64, _vp, _i64, _i64p, _i64p, _vp, _vp,
                                                  _vp, _i64, _i64, _i64, _i64, _vp, _i64, _i64,
                                                  _i64p, _i32, _i32, _vp],
    "sb_rope_correct_k": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64p,
                          _i64p, _i32, _vp],
    "sb_rope_correct_k_distinct": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64p,
                                   _i32, _vp],
    "sb_apply_rope_delta_inplace": [_vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _i64,
                                    _i64, _i64, _i64p, _i32, _vp],
    "sb_apply_rope_delta_inplace_host": [_vp, _vp, _i32p, _i32p, _i64, _i64, _vp, _i64, _i64,
                                         _i64, _i64, _i64, _i64p, _i32, _vp],
    "sb_apply_rope_deltas_inplace_layers": [_vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _i64,
                                            _i64, _i64, _i64, _i64p, _i32, _vp],
    "sb_apply_rope_deltas_inplace_layers_host": [_vp, _i64, _vp, _i32p, _i32p, _i64, _vp, _i64,
                                                 _i64, _i64, _i64, _i64, _i64p, _i32, _vp],
    "sb_permute_paged_kv_with_rope": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                      _i64, _i64, _i64p, _i32, _vp],
    "sb_nope_permute_paged_kv": [_vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _i64,
                                 _i64, _i64, _i64, _i64, _i64p, _i32, _vp],
    "sb_permute_paged_kv_with_rope_layers": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                             _i64, _i64, _i64, _i64, _i64p, _i32, _vp],
    "sb_nope_permute_paged_kv_layers": [_vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp,
                                        _vp, _i64, _i64, _i64, _i64, _i64, _i64p, _i32, _vp],
    "sb_partial_prefill_attention": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                     _f32, _i64p, _i64p, _i64p, _i64p, _i32, _vp],
    "sb_partial_attention_paged": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                   _i64, _i64, _i64, _f32, _i64p, _i64p, _i64p, _i32, _vp],
    "sb_partial_attention_paged_planned": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp,
                                           _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                           _f32, _i64p, _i64p, _i64p, _i32, _vp],
    "sb_partial_attention_paged_varlen": [_vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64p, _i64p,
                                          _vp, _i64, _i64, _i64, _i64, _i64, _i64, _f32,
                                          _i64p, _i64p, _i64p, _i32, _vp],
    "sb_partial_attention_paged_noalloc": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                           _i64, _i64, _i64, _f32, _i64p, _i64p, _i64p, _i32,
                                           _vp],
    "sb_masked_qkv_projection": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                 _i64, _i64, _i32, _vp],
    "sb_qkv_projection_paged": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                _vp, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                _i64p, _i32, _vp],
    "sb_qkv_gather_rows": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i32, _vp],
    "sb_qkv_epilogue_paged": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp,
                              _vp, _i64, _i64, _i64, _i64, _i64, _i64p, _i32, _vp],
    "sb_device_copy": [_vp, _vp, _i64, _vp],
    "sb_kernel_timing_enable": [_i32],
    "sb_kernel_timing_read": [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), _i64p],
}

# Size queries (return int64_t, not a status code).
SIZE_QUERIES: dict[str, list] = {
    "sb_partial_prefill_attention_workspace_size": [_i64, _i64, _i64, _i32],
    "sb_partial_attention_paged_workspace_size": [_i64, _i64, _i64, _i64, _i64, _i64, _i32],
    "sb_partial_attention_paged_varlen_workspace_size": [_i64, _i64p, _i64p, _i64, _i64, _i64,
                                                         _i64, _i32],
    "sb_partial_attention_paged_noalloc_max_scratch": [],
    "sb_partial_attention_paged_plan": [_i32p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32p,
                                        _i64],
    "sb_partial_attention_paged_planned_workspace_size": [_i64, _i64, _i64, _i64, _i32, _i32],
    "sb_masked_qkv_projection_workspace_size": [_i64],
    "sb_qkv_projection_paged_workspace_size": [_i64, _i64, _i64, _i64, _i64, _i32],
}

_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def _load() -> ctypes.CDLL:
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        _load_error = (
            f"{LIB_PATH} is missing; build it with `python -m semblend_amd._build` "
            "(hipcc, gfx950)"
        )
        raise RuntimeError(_load_error)
    try:
        lib = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
    except OSError as exc:  # pragma: no cover - depends on the runtime image
        _load_error = f"failed to load {LIB_PATH}: {exc}"
        raise RuntimeError(_load_error) from exc
    try:
        lib.sb_version.restype = ctypes.c_char_p
        lib.sb_version.argtypes = []
        lib.sb_last_error_string.restype = ctypes.c_char_p
        lib.sb_last_error_string.argtypes = []
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = argtypes
        for name, argtypes in SIZE_QUERIES.items():
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int64
            fn.argtypes = argtypes
    except AttributeError as exc:
        _load_error = (f"{LIB_PATH} does not export the expected C ABI ({exc}); rebuild it "
                       "with `python -m semblend_amd._build`")
        raise RuntimeError(_load_error) from exc
    _lib = lib
    return lib


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError if it cannot be loaded."""
    return _load()


def available() -> bool:
    try:
        _load()
        return True
    except RuntimeError:
        return False


def version() -> str:
    return lib().sb_version().decode()


def size_query(name: str, *args) -> int:
    return int(getattr(lib(), name)(*args))


def call(name: str, *args) -> None:
    """Invoke an entry point and turn a nonzero status into RuntimeError."""
    rc = getattr(lib(), name)(*args)
    if rc != SB_OK:
        msg = lib().sb_last_error_string().decode()
        kind = "invalid argument" if rc == SB_ERR_INVALID_ARGUMENT else f"hip error {rc}"
        raise RuntimeError(f"{name} failed ({kind}): {msg}")


# ------------------------------------------------------------------------------------------
# Argument helpers
# ------------------------------------------------------------------------------------------

def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def strides(t: torch.Tensor, dims: tuple[int, ...] | None = None):
    s = t.stride() if dims is None else tuple(t.stride(d) for d in dims)
    return (ctypes.c_int64 * len(s))(*s)


def i32_array(values) -> ctypes.Array:
    """Host int32 array for arguments the library reads on the host."""
    return (ctypes.c_int32 * len(values))(*values)


def i64_array(values) -> ctypes.Array:
    vals = list(values)
    return (ctypes.c_int64 * len(vals))(*vals)


def dtype_code(t: torch.Tensor) -> int:
    try:
        return SB_DTYPE[t.dtype]
    except KeyError:
        raise TypeError(
            f"unsupported dtype {t.dtype}; the HIP kernels take float32, float16 or bfloat16"
        ) from None


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one HIP device; CPU tensors are rejected (no CPU path)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "semblend_amd runs on MI355X (HIP) device tensors only; got a tensor on "
                f"{t.device}. Move the KV cache and inputs to the GPU."
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no device tensor given")
    return dev


# torch's own raw accessors (what its compiler's generated code uses): a plain int for the
# current stream and device, without building Python stream or device objects per launch.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_current_index = getattr(torch._C, "_cuda_getDevice", None)


def _index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def stream_handle(device: torch.device) -> int:
    """The current stream of ``device`` as a raw handle for the C ABI."""
    if _raw_stream is not None:
        return _raw_stream(_index(device))
    return torch.cuda.current_stream(device).cuda_stream


def on_device(device: torch.device):
    """Context that makes ``device`` current for a launch; a no-op when it already is."""
    if _current_index is not None and _current_index() == _index(device):
        return contextlib.nullcontext()
    return torch.cuda.device(device)


# Pinned staging buffers of host-to-device copies recorded into a HIP graph: every replay
# copies from the same host address again, so they are kept for the life of the process.
_CAPTURED_UPLOADS: list[torch.Tensor] = []


def pinned_upload(host: torch.Tensor, device: torch.device) -> torch.Tensor:
    """Device copy of a contiguous host tensor, staged through pinned memory and enqueued on
    the current stream without blocking the host (torch's pinned-memory cache keeps the
    staging block until the copy has run, then reuses it).

    While the current stream is capturing a HIP graph no pinned memory can be allocated, and a
    captured copy reads its host buffer again at every replay: a host tensor that is already
    pinned is copied and kept for the life of the process (so the replays read the values it
    holds now, as long as the caller does not write to it), anything else raises."""
    if torch.cuda.is_current_stream_capturing():
        if not host.is_pinned():
            raise RuntimeError(
                "host index data cannot be uploaded while the stream is capturing a HIP graph: "
                "pass device tensors (or pinned host tensors), or make the call once before "
                "capture")
        _CAPTURED_UPLOADS.append(host)
        return host.to(device, non_blocking=True)
    return host.pin_memory().to(device, non_blocking=True)


def upload_index(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    """int32 contiguous device copy of a host index tensor (``pinned_upload``)."""
    host = t.to(torch.int32).contiguous()
    if host.numel() == 0:
        return torch.empty(host.shape, dtype=torch.int32, device=device)
    return pinned_upload(host, device)


def as_index(t, device: torch.device) -> torch.Tensor:
    """int32 contiguous device copy of an index tensor or sequence (no copy if already so);
    host data is uploaded without blocking the host."""
    if (isinstance(t, torch.Tensor) and t.dtype == torch.int32 and t.dim() == 1 and t.is_cuda
            and t.get_device() == _index(device) and t.is_contiguous()):
        return t
    if not isinstance(t, torch.Tensor):
        t = torch.as_tensor(list(t), dtype=torch.int32)
    if t.device.type == "cpu":
        return upload_index(t, device).reshape(-1)
    if t.device != device:
        t = t.to(device)
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous().reshape(-1)


def rows_repeat(positions, donor_index=None, sync: bool = False) -> bool:
    """Whether some donor row is the source of more than one pair: a position that occurs
    twice (with the same donor, when ``donor_index`` is given). Host data is checked on the
    host; device tensors only when ``sync`` allows one device-to-host read, and are otherwise
    taken as distinct. Only the scatters' load policy depends on the answer, not their
    results."""
    on_dev = any(isinstance(x, torch.Tensor) and x.device.type != "cpu"
                 for x in (positions, donor_index))
    if on_dev and not sync:
        return False
    if not isinstance(positions, torch.Tensor):
        positions = torch.as_tensor(list(positions) if not hasattr(positions, "__array__")
                                    else positions)
    key = positions.reshape(-1).to(torch.int64)
    n = key.numel()
    if n < 2:
        return False
    if donor_index is not None:
        if not isinstance(donor_index, torch.Tensor):
            donor_index = torch.as_tensor(list(donor_index) if not hasattr(
                donor_index, "__array__") else donor_index)
        idx = donor_index.reshape(-1).to(device=key.device, dtype=torch.int64)
        key = idx * (1 << 32) + (key & 0xFFFFFFFF)
    return int(torch.unique(key).numel()) < n


def scatter_flags(repeated: bool) -> int:
    return SB_SCATTER_REPEATED_DONOR_ROWS if repeated else 0


_ADDR_TABLES: dict[tuple, torch.Tensor] = {}
_ADDR_TABLES_MAX = 64
# Tables used by a launch recorded into a HIP graph: a replay may come at any time, so these
# are never evicted (with the pinned host copy a captured upload reads from).
_CAPTURED_TABLES: dict[tuple, tuple[torch.Tensor, torch.Tensor | None]] = {}


def address_table(tensors, device: torch.device) -> torch.Tensor:
    """Device int64 array of the tensors' base addresses (the per-layer tables of the
    multi-layer entry points).

    Tables are cached by (device, addresses), so repeated calls over the same layer tensors
    enqueue no host-to-device copy; a new table is copied from pinned memory without blocking
    the host. Keying by the addresses themselves keeps a cached table correct even when the
    tensors are freed and others reuse the memory. Lifetime: a table is marked as used on
    the current stream at every call, so evicting it from the bounded cache never releases
    memory that a kernel enqueued on another stream still reads; a table requested while the
    current stream is capturing a HIP graph is kept for the life of the process, since the
    graph holds its raw address. Callers that repeat one launch should prefer the prepared
    forms (``rope_correction.prepare_scatter_paged_layers``), which own their tables.
    """
    key = (device, tuple(t.data_ptr() for t in tensors))
    capturing = torch.cuda.is_current_stream_capturing()
    kept = _CAPTURED_TABLES.get(key)
    if kept is not None:
        return kept[0]
    tab = _ADDR_TABLES.get(key)
    host = None
    if tab is None:
        if len(_ADDR_TABLES) >= _ADDR_TABLES_MAX:
            _ADDR_TABLES.pop(next(iter(_ADDR_TABLES)))
        host = torch.tensor(key[1], dtype=torch.int64).pin_memory()
        tab = host.to(device, non_blocking=True)
        if not capturing:
            _ADDR_TABLES[key] = tab
    if capturing:
        _ADDR_TABLES.pop(key, None)
        _CAPTURED_TABLES[key] = (tab, host)
    else:
        tab.record_stream(torch.cuda.current_stream(device))
    return tab


def device_copy(dst: torch.Tensor, src: torch.Tensor) -> None:
    """``dst <- src`` (same byte count, contiguous, 16-byte aligned) through the library's
    flat copy kernel on the current stream: the achievable-bandwidth reference that the row
    movers are measured against."""
    if not (dst.is_contiguous() and src.is_contiguous()):
        raise ValueError("device_copy takes contiguous tensors")
    nbytes = dst.numel() * dst.element_size()
    if nbytes != src.numel() * src.element_size():
        raise ValueError("device_copy: byte counts differ")
    dev = require_device(dst, src)
    with on_device(dev):
        call("sb_device_copy", dst.data_ptr(), src.data_ptr(), nbytes, stream_handle(dev))


def kernel_timing(enable: bool) -> None:
    """Start (clearing the log) or stop attaching HIP timing events to the library's kernel
    launches (stamped by the runtime with each kernel's start and end)."""
    call("sb_kernel_timing_enable", 1 if enable else 0)


def kernel_time(kernel: str) -> tuple[float, int]:
    """(total milliseconds, launches) logged for one kernel since timing was last enabled."""
    total = ctypes.c_double(0.0)
    n = ctypes.c_int64(0)
    call("sb_kernel_timing_read", kernel.encode(), ctypes.byref(total), ctypes.byref(n))
    return total.value, n.value
