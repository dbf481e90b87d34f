"""The native module, re-presented over the C ABI of libmicroinfer_hip.so.

Drop-in for the reference's pybind11 module `_microinfer` and its submodule
`_microinfer.device` (src/core_kernels/bindings.cpp:427-669,
bindings_device.cpp:251-993): the same names, argument meanings, defaults,
exception classes and message keywords, on top of the `extern "C"` entry
points declared in include/microinfer_hip.h. ctypes releases the GIL around
every foreign call, as the reference's bindings release it around device
work (ADR-0012).

There is no fallback: if the library is missing this module raises on
import, and every device call goes to the HIP kernels.
"""

from __future__ import annotations

import ctypes as C
import enum
import os
import weakref
from pathlib import Path
from types import SimpleNamespace

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "libmicroinfer_hip.so"
if not _LIB_PATH.exists():
    raise ImportError(f"{_LIB_PATH} is not built: run `python build.py` in "
                      f"{_LIB_PATH.parent.parent} (or __graft_entry__.build()); there is no "
                      f"CPU fallback")
lib = C.CDLL(str(_LIB_PATH))

_vp, _sz, _i, _f, _d = C.c_void_p, C.c_size_t, C.c_int, C.c_float, C.c_double
_ll = C.c_longlong
_ip, _szp, _fp = C.POINTER(C.c_int), C.POINTER(C.c_size_t), C.POINTER(C.c_float)


class _Layout(C.Structure):
    _fields_ = [("bits", C.c_int), ("key_codes", _sz), ("value_codes", _sz), ("key_scales", _sz),
                ("key_zeros", _sz), ("value_scales", _sz), ("value_zeros", _sz),
                ("metadata_bytes", _sz), ("page_bytes", _sz), ("effective_bits", C.c_double)]


class _ModelShape(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("layers", "hidden", "intermediate", "heads", "kv_heads",
                                        "head_dim", "vocab")] + \
               [("rms_eps", C.c_float), ("rope_theta", C.c_double)]


_LAYER_TENSORS = ("input_norm", "q_w", "q_b", "k_w", "k_b", "v_w", "v_b", "o_w", "post_norm",
                  "gate_w", "up_w", "down_w")


class _LayerWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in _LAYER_TENSORS]


class _KVInfo(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("layers", "page_tokens", "kv_heads", "head_dim",
                                        "pages_per_layer", "capacity_tokens", "tier", "halves",
                                        "storage_tier", "seals", "born_at_one_tier")] + \
               [(n, _sz) for n in ("page_bytes", "kv_width", "shadow_count", "shadow_bytes")]


def _sig(name, *args, restype=C.c_int):
    fn = getattr(lib, name)
    fn.argtypes = list(args)
    fn.restype = restype
    return fn


# Every exported entry point's signature (include/microinfer_hip.h).
SIGNATURES = {
    "mi_last_error": ((), C.c_char_p), "mi_build_info": ((), C.c_char_p),
    "mi_device_count": ((_ip,), C.c_int), "mi_device_name": ((C.c_char_p, _sz), C.c_int),
    "mi_runtime_version": ((_ip,), C.c_int),
    "mi_host_alloc": ((C.POINTER(_vp), C.POINTER(_vp), _sz), C.c_int),
    "mi_kv_store_at": ((_vp, _i, _vp, _vp, _vp), C.c_int),
    "mi_kv_attention_at": ((_vp, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp), C.c_int),
    "mi_kv_stored_on_device": ((_vp, _i), C.c_int),
    "mi_kv_rope_store": ((_vp, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _f), C.c_int),
    "mi_kv_attend_row": ((_vp, _i, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _f),
                         C.c_int),
    "mi_decode_step_create": ((C.POINTER(_vp), _vp, C.POINTER(_ModelShape), _vp, _vp, _vp,
                               C.POINTER(_LayerWeights), _vp, _i), C.c_int),
    "mi_decode_step_destroy": ((_vp,), C.c_int),
    "mi_decode_step_run": ((_vp, _i, _i, _i, C.POINTER(C.c_int32), C.POINTER(_d)), C.c_int),
    "mi_decode_step_run_eager": ((_vp, _i, _i, _i, C.POINTER(C.c_int32), C.POINTER(_d)),
                                 C.c_int),
    "mi_decode_step_logits": ((_vp, _fp, _sz), C.c_int),
    "mi_decode_step_prefill": ((_vp, C.POINTER(C.c_int32), _i, _i, _i, C.POINTER(C.c_int32),
                                C.POINTER(_d)), C.c_int),
    "mi_decode_step_launches": ((_vp, _ip), C.c_int),
    "mi_decode_step_plans": ((_vp, _ip, _sz, _szp), C.c_int),
    "mi_random_half": ((_vp, _sz, C.c_ulonglong, _f), C.c_int),
    "mi_host_free": ((_vp,), C.c_int),
    "mi_device_pci_bus_id": ((C.c_char_p, _sz), C.c_int), "mi_memory_info": ((_szp, _szp), C.c_int),
    "mi_granule_bytes": ((_szp,), C.c_int), "mi_malloc": ((C.POINTER(_vp), _sz), C.c_int),
    "mi_free": ((_vp,), C.c_int), "mi_memcpy": ((_vp, _vp, _sz, _i), C.c_int),
    "mi_memset": ((_vp, _i, _sz), C.c_int), "mi_synchronize": ((), C.c_int),
    "mi_event_create": ((C.POINTER(_vp),), C.c_int), "mi_event_destroy": ((_vp,), C.c_int),
    "mi_event_record": ((_vp, _vp), C.c_int), "mi_event_elapsed_ms": ((_vp, _vp, _fp), C.c_int),
    "mi_stream_create": ((C.POINTER(_vp),), C.c_int), "mi_stream_destroy": ((_vp,), C.c_int),
    "mi_stream_synchronize": ((_vp,), C.c_int), "mi_set_stream": ((_vp,), C.c_int),
    "mi_graph_begin": ((_vp,), C.c_int), "mi_graph_end": ((_vp, C.POINTER(_vp)), C.c_int),
    "mi_graph_launch": ((_vp, _vp), C.c_int), "mi_graph_destroy": ((_vp,), C.c_int),
    "mi_half_bits_from_double": ((_d,), C.c_uint16),
    "mi_scale_bits_of": ((_f, _f, _i), C.c_uint16),
    "mi_quantised_page_layout": ((_i, _i, _i, _i, C.POINTER(_Layout)), C.c_int),
    "mi_fp16_page_bytes": ((_i, _sz), _sz),
    "mi_quantise_page": ((_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp), C.c_int),
    "mi_quantise_pages": ((_vp, _vp, _i, _i, _i, _i, _i, _vp), C.c_int),
    "mi_dequantise_page": ((_vp, _vp, _vp, _i, _i, _i, _i, _vp), C.c_int),
    "mi_attention_partials_floats": ((_i,), _sz),
    "mi_attention_split": ((_i, _i, _i, _i, _i, _ip, _ip), C.c_int),
    "mi_attention": ((_vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _vp, _vp), C.c_int),
    "mi_attention_paged": ((_vp, _vp, _i, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _vp, _vp, _vp),
                           C.c_int),
    "mi_attention_paged_causal": ((_vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _i,
                                   _i, _i, _i, _i, _vp, _vp, _f, _vp, _vp), C.c_int),
    "mi_attention_paged_causal_noalloc": ((_vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _i, _i,
                                           _i, _i, _vp, _vp, _f, _vp), C.c_int),
    "mi_copy_pages": ((_vp, _vp, _sz, _i, _vp), C.c_int),
    "mi_store_pages": ((_vp, _vp, _vp, _i, _sz, _i, _i, _vp), C.c_int),
    "mi_fill_f32": ((_vp, _sz, _f, _vp), C.c_int),
    "mi_fold_scores": ((_vp, _vp, _i, _i, _f, _vp), C.c_int),
    "mi_rope": ((_vp, _vp, _vp, _i, _i, _i, _d, _vp), C.c_int),
    "mi_rope_table_fill": ((_vp, _i, _i, _d, _vp), C.c_int),
    "mi_rope_from_table": ((_vp, _vp, _vp, _i, _vp, _i, _i, _i, _vp), C.c_int),
    "mi_rmsnorm": ((_vp, _i, _vp, _vp, _i, _i, _f, _vp), C.c_int),
    "mi_swiglu": ((_vp, _vp, _vp, _sz, _vp), C.c_int),
    "mi_add": ((_vp, _vp, _vp, _sz, _vp), C.c_int),
    "mi_driver_version": ((_ip,), C.c_int),
    "mi_linear": ((_vp, _vp, _vp, _vp, _i, _i, _i, _vp), C.c_int),
    "mi_linear_f32": ((_vp, _vp, _vp, _i, _i, _i, _i, _vp), C.c_int),
    "mi_embed": ((_vp, _i, _vp, _vp, _i, _i, _i, _vp), C.c_int),
    "mi_argmax_rows": ((_vp, _i, _i, _vp, _vp), C.c_int),
    "mi_scratch_elements": ((_i, _i, _szp), C.c_int),
    "mi_logits": ((_vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp), C.c_int),
    "mi_greedy": ((_vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp), C.c_int),
    "mi_cache_create": ((_szp, _szp, C.POINTER(_vp)), C.c_int),
    "mi_cache_destroy": ((_vp,), None),
    "mi_cache_allocate": ((_vp, _i, _i, _i), C.c_int),
    "mi_cache_free": ((_vp, _i, _i), C.c_int),
    "mi_cache_free_pages": ((_vp, _ip, _sz), C.c_int),
    "mi_cache_replace": ((_vp, _i, _i, _i, _i), C.c_int),
    "mi_cache_replace_pages": ((_vp, _ip, _sz), C.c_int),
    "mi_cache_write": ((_vp, _i, _i, _vp, _sz), C.c_int),
    "mi_cache_read": ((_vp, _i, _i, _vp, _sz), C.c_int),
    "mi_cache_locate": ((_vp, _i, _i, _ip, _szp), C.c_int),
    "mi_cache_contains": ((_vp, _i, _i, _ip), C.c_int),
    "mi_cache_pages": ((_vp, _i, _ip, _sz, _szp), C.c_int),
    "mi_cache_page_bytes": ((_vp, _i, _szp), C.c_int),
    "mi_cache_reserved_bytes": ((_vp, _i, _szp), C.c_int),
    "mi_cache_mapped_bytes": ((_vp, _i, _szp), C.c_int),
    "mi_cache_keep_spare_granules": ((_vp, _i, _sz), C.c_int),
    "mi_cache_drain_releases": ((_vp,), C.c_int),
    "mi_cache_spare_granules": ((_vp, _i, _szp), C.c_int),
    "mi_cache_granule_bytes": ((_vp, _szp), C.c_int),
    "mi_debug_fail_next_granules": ((_i,), C.c_int),
    "mi_shadows_create": ((_sz, C.POINTER(_vp)), C.c_int),
    "mi_shadows_destroy": ((_vp,), None),
    "mi_shadows_take": ((_vp, _i, _i, _vp), C.c_int),
    "mi_shadows_contains": ((_vp, _i, _i, _ip), C.c_int),
    "mi_shadows_read": ((_vp, _i, _i, _vp, _sz), C.c_int),
    "mi_shadows_count": ((_vp, _szp), C.c_int),
    "mi_shadows_bytes": ((_vp, _szp), C.c_int),
    "mi_scores_create": ((_i, _i, _f, C.POINTER(_vp)), C.c_int),
    "mi_scores_destroy": ((_vp,), None),
    "mi_scores_fold": ((_vp, _i, _vp, _i, _i), C.c_int),
    "mi_scores_download": ((_vp, _vp, _sz), C.c_int),
    "mi_scores_upload": ((_vp, _vp, _i, _i), C.c_int),
    "mi_scores_layer_row": ((_vp, _i, C.POINTER(_vp)), C.c_int),
    "mi_scores_info": ((_vp, _ip, _ip, _fp, _szp), C.c_int),
    "mi_rope_table_create": ((_i, _d, C.POINTER(_vp)), C.c_int),
    "mi_rope_table_destroy": ((_vp,), None),
    "mi_rope_table_cover": ((_vp, _i), C.c_int),
    "mi_rope_table_info": ((_vp, _ip, C.POINTER(_vp)), C.c_int),
    "mi_kv_create": ((_vp, _i, _i, _i, _i, _i, _i, _ip, _ip, _i, _i, C.POINTER(_vp)), C.c_int),
    "mi_kv_destroy": ((_vp,), None),
    "mi_kv_seals_for": ((_i, _ip, _ip, _i, _i, _ip), C.c_int),
    "mi_kv_reserve": ((_vp, _i), C.c_int),
    "mi_kv_store": ((_vp, _i, _vp, _vp, _i, _i), C.c_int),
    "mi_kv_attention": ((_vp, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _f,
                         _vp), C.c_int),
    "mi_kv_attention_layers": ((_vp, _i, _i, _vp, _ll, _vp, _ll, _i, _i, _i, _i, _vp, _vp, _ll,
                                _vp, _ll, _vp, _ll, _f), C.c_int),
    "mi_kv_attention_kept": ((_vp, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp), C.c_int),
    "mi_kv_fold_kept": ((_vp, _vp, _ll, _vp, _ll, _f), C.c_int),
    "mi_kv_downgrade": ((_vp, _i, _i, _i), C.c_int),
    "mi_kv_upgrade": ((_vp, _i, _i, _i), C.c_int),
    "mi_kv_move_pages": ((_vp, _ip, _sz), C.c_int),
    "mi_kv_pin_shadows": ((_vp, _sz), C.c_int),
    "mi_kv_evict": ((_vp, _i, _i), C.c_int),
    "mi_kv_mask": ((_vp, _i, _i), C.c_int),
    "mi_kv_page_tier": ((_vp, _i, _i, _ip), C.c_int),
    "mi_kv_has_shadow": ((_vp, _i, _i, _ip), C.c_int),
    "mi_kv_shadow": ((_vp, _i, _i, _vp, _sz), C.c_int),
    "mi_kv_page_tiers": ((_vp, _vp, _sz), C.c_int),
    "mi_kv_flags": ((_vp, _i, _vp, _sz), C.c_int),
    "mi_kv_info_get": ((_vp, C.POINTER(_KVInfo)), C.c_int),
    "mi_kv_birth_tier": ((_vp, _i, _i, _ip), C.c_int),
    "mi_kv_last_move": ((_vp, _ip, _ip, _szp, C.POINTER(C.c_double)), C.c_int),
    "mi_kv_last_batch": ((_vp, _ip, _szp, _szp, C.POINTER(C.c_double)), C.c_int),
    "mi_kv_last_batch_phases": ((_vp, C.POINTER(C.c_double)), C.c_int),
}
for _name, (_args, _res) in SIGNATURES.items():
    _sig(_name, *_args, restype=_res)


# -- errors (bindings.cpp:546-554) ---------------------------------------------------

class PageNotFound(KeyError):
    """A page the page table does not hold."""

    def __str__(self):
        return str(self.args[0]) if self.args else ""


class OpenPage(ValueError):
    """A page still being filled cannot be quantised."""


class OutOfMemory(MemoryError):
    """The device has no memory for a granule or a buffer."""


class DeviceError(RuntimeError):
    """A HIP runtime error."""


_ERRORS = {1: ValueError, 2: IndexError, 3: PageNotFound, 4: OpenPage, 5: OutOfMemory,
           6: RuntimeError, 7: ValueError, 8: DeviceError}


def _check(status: int) -> None:
    if status != 0:
        message = (lib.mi_last_error() or b"").decode(errors="replace")
        raise _ERRORS.get(status, RuntimeError)(message)


# -- tiers ----------------------------------------------------------------------------

class Tier(enum.IntEnum):
    """Precision tier, highest first (paged_kv_cache.h:16-25)."""
    FP16 = 0
    INT8 = 1
    INT4 = 2
    INT2 = 3


def _tier(t) -> int:
    value = int(t)
    if value not in (0, 1, 2, 3):
        raise ValueError(f"tier {value} is not one of the four")
    return value


# -- device memory ------------------------------------------------------------------------

def _malloc(nbytes: int) -> int:
    p = _vp()
    _check(lib.mi_malloc(C.byref(p), nbytes))
    return p.value or 0


def _free(ptr: int) -> None:
    if ptr:
        lib.mi_free(ptr)


class _Storage:
    """An allocation, freed when the last object holding it goes."""

    def __init__(self, nbytes: int):
        self.nbytes = nbytes
        self.ptr = _malloc(nbytes)
        weakref.finalize(self, _free, self.ptr)


def _h2d(ptr: int, host: np.ndarray) -> None:
    host = np.ascontiguousarray(host)
    if host.nbytes:
        _check(lib.mi_memcpy(ptr, host.ctypes.data, host.nbytes, 0))


def _d2h(host: np.ndarray, ptr: int) -> None:
    if host.nbytes:
        _check(lib.mi_memcpy(host.ctypes.data, ptr, host.nbytes, 1))


class DeviceTensor:
    """fp16 on the device (device_tensor.cu:14-152): in an allocation of its
    own, or at an offset into a DeviceArena, which it keeps alive."""

    def __init__(self, count: int, storage: _Storage | None = None, offset: int = 0):
        self._storage = storage if storage is not None else _Storage(2 * count)
        self._ptr = self._storage.ptr + offset
        self.numel = count

    @property
    def address(self) -> int:
        return self._ptr

    @property
    def nbytes(self) -> int:
        return 2 * self.numel

    def to_numpy(self) -> np.ndarray:
        out = np.empty(self.numel, np.float16)
        _d2h(out, self._ptr)
        return out.astype(np.float32)

    def raw(self) -> np.ndarray:
        """The fp16 bits, unwidened."""
        out = np.empty(self.numel, np.float16)
        _d2h(out, self._ptr)
        return out


def upload_fp16(host) -> DeviceTensor:
    """A float32 array to the device as fp16, rounded on the host."""
    h = np.ascontiguousarray(host, np.float32).astype(np.float16).reshape(-1)
    t = DeviceTensor(h.size)
    _h2d(t.address, h)
    return t


weight_alignment = 256


class HostBuffer:
    """Pinned host memory mapped for the device (beyond the reference):
    `address` is what kernels use, `array` the host's view (uint8)."""

    def __init__(self, nbytes: int):
        h, dv = _vp(), _vp()
        _check(lib.mi_host_alloc(C.byref(h), C.byref(dv), nbytes))
        self._host, self.address, self.nbytes = h.value, dv.value, nbytes
        weakref.finalize(self, lib.mi_host_free, self._host)
        self.array = np.ctypeslib.as_array((C.c_uint8 * nbytes).from_address(self._host))


class DeviceArena:
    """One device allocation that many DeviceTensors refer into."""

    def __init__(self, nbytes: int):
        self._storage = _Storage(nbytes)
        self.nbytes = nbytes

    @property
    def address(self) -> int:
        return self._storage.ptr

    def put(self, offset: int, host) -> DeviceTensor:
        h = np.ascontiguousarray(host, np.float32).astype(np.float16).reshape(-1)
        if offset % weight_alignment != 0 or offset < 0 or offset + h.nbytes > self.nbytes:
            raise ValueError(f"offset {offset} for {h.nbytes} bytes: offsets are multiples of "
                             f"{weight_alignment} within the arena's {self.nbytes} bytes")
        t = DeviceTensor(h.size, self._storage, offset)
        _h2d(t.address, h)
        return t


def device_name() -> str:
    buf = C.create_string_buffer(256)
    _check(lib.mi_device_name(buf, 256))
    return buf.value.decode()


def device_pci_bus_id() -> str:
    """The current device's PCI bus id, as amdsmi names GPUs."""
    buf = C.create_string_buffer(64)
    _check(lib.mi_device_pci_bus_id(buf, 64))
    return buf.value.decode()


def hip_runtime_version() -> int:
    v = C.c_int()
    _check(lib.mi_runtime_version(C.byref(v)))
    return v.value


def driver_version() -> int:
    """The HIP driver's version (the reference's cuda_driver_version)."""
    v = C.c_int()
    _check(lib.mi_driver_version(C.byref(v)))
    return v.value


cuda_driver_version = driver_version


def device_memory_info() -> dict:
    free, total = C.c_size_t(), C.c_size_t()
    _check(lib.mi_memory_info(C.byref(free), C.byref(total)))
    return {"free": free.value, "total": total.value}


def granule_bytes() -> int:
    g = C.c_size_t()
    _check(lib.mi_granule_bytes(C.byref(g)))
    return g.value


class PageCopy:
    """A batch of page copies (page_copy.cu:41-70): nbytes from each device
    address in `sources` to the matching one in `destinations`, the address
    tables uploaded once; launch() enqueues the one batched copy on the null
    stream. No copy may read what another writes."""

    def __init__(self, sources, destinations, nbytes: int):
        src = np.ascontiguousarray(sources, np.uint64).reshape(-1)
        dst = np.ascontiguousarray(destinations, np.uint64).reshape(-1)
        if src.size != dst.size:
            raise ValueError(f"{src.size} sources for {dst.size} destinations")
        self.count, self.nbytes = int(src.size), int(nbytes)
        self._tables = _Storage(max(16 * src.size, 16))
        _h2d(self._tables.ptr, np.concatenate([src, dst]))

    def launch(self) -> None:
        if self.count:
            _check(lib.mi_copy_pages(self._tables.ptr, self._tables.ptr + 8 * self.count,
                                     self.nbytes, self.count, None))


def copy_pages(sources, destinations, nbytes: int) -> None:
    """One batched copy of nbytes per (source, destination), waited for."""
    PageCopy(sources, destinations, nbytes).launch()
    synchronize()


def synchronize() -> None:
    _check(lib.mi_synchronize())


# -- quantised pages (bindings.cpp:358-425) ----------------------------------------------

P_DEFAULT = 32


def quantised_page_layout(tier, kv_heads: int, head_dim: int, page_tokens: int = P_DEFAULT) -> dict:
    out = _Layout()
    _check(lib.mi_quantised_page_layout(_tier(tier), page_tokens, kv_heads, head_dim,
                                        C.byref(out)))
    return {name: getattr(out, name) for name, _ in _Layout._fields_}


def _shape(a) -> str:
    return "(" + ", ".join(str(n) for n in np.shape(a)) + ")"


def quantise_page(keys, values, tier, page_tokens: int = P_DEFAULT) -> np.ndarray:
    keys = np.ascontiguousarray(keys, np.float32)
    values = np.ascontiguousarray(values, np.float32)
    if keys.ndim != 3:
        raise ValueError(f"keys must be 3-D (positions, kv_heads, head_dim), got shape {_shape(keys)}")
    if values.shape != keys.shape:
        raise ValueError(f"values must have the keys' shape {_shape(keys)}, got shape {_shape(values)}")
    filled, kv_heads, head_dim = keys.shape
    layout = quantised_page_layout(tier, kv_heads, head_dim, page_tokens)
    if filled < page_tokens:
        raise OpenPage(f"the page holds {filled} of {page_tokens} positions and is still being "
                       f"filled: a key channel's scale spans the whole page, so the open page "
                       f"stays at FP16")
    if filled > page_tokens:
        raise ValueError(f"{filled} positions do not fit a page of {page_tokens}")
    k = upload_fp16(keys)
    v = upload_fp16(values)
    page = _Storage(layout["page_bytes"])
    _check(lib.mi_quantise_page(k.address, v.address, page.ptr, _tier(tier), page_tokens, filled,
                                kv_heads, head_dim, None))
    out = np.empty(layout["page_bytes"], np.uint8)
    _d2h(out, page.ptr)
    return out


def dequantise_page(page, tier, kv_heads: int, head_dim: int, page_tokens: int = P_DEFAULT):
    layout = quantised_page_layout(tier, kv_heads, head_dim, page_tokens)
    page = np.ascontiguousarray(page, np.uint8)
    if page.ndim != 1 or page.shape[0] != layout["page_bytes"]:
        raise ValueError(f"a page at this tier and shape is {layout['page_bytes']} bytes, got "
                         f"shape {_shape(page)}")
    dev = _Storage(page.nbytes)
    _h2d(dev.ptr, page)
    count = page_tokens * kv_heads * head_dim
    k, v = DeviceTensor(count), DeviceTensor(count)
    _check(lib.mi_dequantise_page(dev.ptr, k.address, v.address, _tier(tier), page_tokens,
                                  kv_heads, head_dim, None))
    shape = (page_tokens, kv_heads, head_dim)
    return k.to_numpy().reshape(shape), v.to_numpy().reshape(shape)


# -- NumPy-in, NumPy-out kernels (bindings.cpp:31-273) --------------------------------------

def rmsnorm(x, weight, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    weight = np.ascontiguousarray(weight, np.float32)
    if x.ndim != 2:
        raise ValueError(f"x must be 2-D (rows, hidden), got ndim={x.ndim}")
    if weight.ndim != 1:
        raise ValueError(f"weight must be 1-D (hidden,), got ndim={weight.ndim}")
    rows, hidden = x.shape
    if weight.shape[0] != hidden:
        raise ValueError(f"weight length {weight.shape[0]} does not match hidden size {hidden}")
    dx, dw, out = upload_fp16(x), upload_fp16(weight), DeviceTensor(x.size)
    _check(lib.mi_rmsnorm(dx.address, 0, dw.address, out.address, rows, hidden, eps, None))
    return out.to_numpy().reshape(x.shape)


def rope(x, positions, theta: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    positions = np.ascontiguousarray(positions, np.int32)
    if x.ndim != 3:
        raise ValueError(f"x must be 3-D (seq, heads, head_dim), got shape {_shape(x)}")
    if positions.ndim != 1 or positions.shape[0] != x.shape[0]:
        raise ValueError(f"positions must be 1-D with one entry per token: x has seq "
                         f"{x.shape[0]}, positions has shape {_shape(positions)}")
    if x.shape[2] % 2 != 0:
        raise ValueError(f"head_dim must be even for rotate-half RoPE, got {x.shape[2]}")
    if not theta > 0.0:
        raise ValueError(f"theta must be positive, got {theta}")
    if (positions < 0).any():
        i = int(np.argmax(positions < 0))
        raise ValueError(f"positions must not be negative, got {positions[i]} at index {i}")
    dx, out = upload_fp16(x), DeviceTensor(x.size)
    pos = DeviceIndex(positions)
    _check(lib.mi_rope(dx.address, pos.address, out.address, x.shape[0], x.shape[1], x.shape[2],
                       theta, None))
    return out.to_numpy().reshape(x.shape)


def swiglu(gate, up) -> np.ndarray:
    gate = np.ascontiguousarray(gate, np.float32)
    up = np.ascontiguousarray(up, np.float32)
    if gate.ndim != 2 or up.ndim != 2:
        raise ValueError(f"gate and up must be 2-D (rows, intermediate), got {_shape(gate)} and "
                         f"{_shape(up)}")
    if gate.shape != up.shape:
        raise ValueError(f"gate {_shape(gate)} and up {_shape(up)} must have the same shape")
    dg, du, out = upload_fp16(gate), upload_fp16(up), DeviceTensor(gate.size)
    _check(lib.mi_swiglu(dg.address, du.address, out.address, gate.size, None))
    return out.to_numpy().reshape(gate.shape)


def linear(x, weight, bias=None) -> np.ndarray:
    """x @ weight.T + bias through hipBLASLt; weight (out_features,
    in_features) as the checkpoint stores it. fp16 operands, fp32
    accumulation, one fp16 rounding on store (bindings.cpp:158-215)."""
    x = np.ascontiguousarray(x, np.float32)
    weight = np.ascontiguousarray(weight, np.float32)
    if x.ndim != 2:
        raise ValueError(f"x must be 2-D (rows, in_features), got shape {_shape(x)}")
    if weight.ndim != 2:
        raise ValueError(f"weight must be 2-D (out_features, in_features), got shape "
                         f"{_shape(weight)}")
    if weight.shape[1] != x.shape[1]:
        raise ValueError(f"weight {_shape(weight)} does not match x {_shape(x)}: weight is "
                         f"(out_features, in_features) and x has in_features {x.shape[1]}")
    if x.shape[1] == 0:
        raise ValueError("in_features must be at least 1")
    if bias is not None:
        bias = np.ascontiguousarray(bias, np.float32)
        if bias.ndim != 1 or bias.shape[0] != weight.shape[0]:
            raise ValueError(f"bias must be 1-D (out_features,) with out_features "
                             f"{weight.shape[0]}, got shape {_shape(bias)}")
    rows, in_features = x.shape
    out_features = weight.shape[0]
    dx, dw = upload_fp16(x), upload_fp16(weight)
    db = upload_fp16(bias) if bias is not None else None
    out = DeviceTensor(rows * out_features)
    _check(lib.mi_linear(dx.address, dw.address, db.address if db is not None else None,
                         out.address, rows, in_features, out_features, None))
    return out.to_numpy().reshape(rows, out_features)


def attention(q, k, v, k_bias=None, theta: float = 0.0) -> np.ndarray:
    q, k, v = (np.ascontiguousarray(a, np.float32) for a in (q, k, v))
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError(f"q, k and v must be 3-D (tokens, heads, head_dim), got {_shape(q)}, "
                         f"{_shape(k)}, {_shape(v)}")
    if k.shape != v.shape:
        raise ValueError(f"k {_shape(k)} and v {_shape(v)} must have the same shape")
    if q.shape[2] != k.shape[2]:
        raise ValueError(f"q has head_dim {q.shape[2]} and k has head_dim {k.shape[2]}")
    if q.shape[0] > k.shape[0]:
        raise ValueError(f"seq_q {q.shape[0]} exceeds seq_k {k.shape[0]}: queries align to the "
                         f"last keys, so there must be at least as many keys as queries")
    if k_bias is not None:
        k_bias = np.ascontiguousarray(k_bias, np.float32)
        if k_bias.ndim != 2 or k_bias.shape != k.shape[1:]:
            raise ValueError(f"k_bias must be (kv_heads, head_dim) = ({k.shape[1]}, {k.shape[2]}), "
                             f"got {_shape(k_bias)}")
        if not theta > 0.0:
            raise ValueError(f"theta must be positive when k_bias is given, got {theta}")
    seq_q, heads, hd = q.shape
    seq_k, kv_heads, _ = k.shape
    out = DeviceTensor(q.size)
    dq, dk, dv = upload_fp16(q), upload_fp16(k), upload_fp16(v)
    partials = FloatTensor(_attention_partials(hd))
    table = None
    bias = None
    if k_bias is not None:
        table = RopeTable(hd, theta)
        table.cover(seq_k)
        bias = upload_fp16(k_bias)
    _check(lib.mi_attention(dq.address, dk.address, dv.address, bias.address if bias else None,
                            table._data() if table else None, table.positions if table else 0,
                            out.address, seq_q, seq_k, heads, kv_heads, hd, partials.address, None))
    return out.to_numpy().reshape(q.shape)


attention_tiles = {"query": 16, "key": 32}


# -- the device surface (bindings_device.cpp) --------------------------------------------

class Span:
    """A run of fp16 elements in a DeviceTensor; holds the tensor."""

    def __init__(self, tensor, offset: int = 0, count: int | None = None):
        if isinstance(tensor, Span):
            base, start, n = tensor.owner, tensor.offset, tensor.count
        else:
            base, start, n = tensor, 0, tensor.numel
        count = n - offset if count is None else count
        if offset < 0 or count < 0 or offset > n or count > n - offset:
            raise ValueError(f"view [{offset}, {offset + count}) of a tensor of {n} elements")
        self.owner, self.offset, self.count = base, start + offset, count

    @property
    def address(self) -> int:
        return self.owner.address + 2 * self.offset

    def to_numpy(self) -> np.ndarray:
        out = np.empty(self.count, np.float16)
        _d2h(out, self.address)
        return out.astype(np.float32)


def _span(x) -> Span | None:
    if x is None:
        return None
    return x if isinstance(x, Span) else Span(x)


def _need(span, count: int, what: str) -> int:
    if span.count < count:
        held = span.count
        raise ValueError(f"{what} holds {held}, and the operation needs {count}")
    return span.address


def _non_negative(value: int, what: str) -> None:
    if value < 0:
        raise ValueError(f"{what} must not be negative, got {value}")


class FloatTensor:
    """fp32 on the device (the residual stream, masses, partials)."""

    def __init__(self, count: int):
        self._storage = _Storage(4 * count)
        self.numel = count

    @property
    def address(self) -> int:
        return self._storage.ptr

    @property
    def nbytes(self) -> int:
        return 4 * self.numel

    def count(self) -> int:
        return self.numel

    def to_numpy(self) -> np.ndarray:
        out = np.empty(self.numel, np.float32)
        _d2h(out, self.address)
        return out


class DeviceIndex:
    """int32 on the device: token ids or positions."""

    def __init__(self, host):
        h = np.ascontiguousarray(host, np.int32).reshape(-1)
        self._storage = _Storage(max(4 * h.size, 4))
        self.count = h.size
        _h2d(self._storage.ptr, h)

    @property
    def address(self) -> int:
        return self._storage.ptr


def _attention_partials(head_dim: int) -> int:
    return int(lib.mi_attention_partials_floats(head_dim))


def _floats(t: FloatTensor | None, count: int, what: str):
    if t is None:
        return None
    if t.numel < count:
        raise ValueError(f"{what} needs {count} floats; got {t.numel}")
    return t.address


class RopeTable:
    """cos and sin of every RoPE angle per position, fp32 on the device
    (rope_table.h:25-44)."""

    def __init__(self, head_dim: int, theta: float):
        h = _vp()
        _check(lib.mi_rope_table_create(head_dim, theta, C.byref(h)))
        self._h = h.value
        self.head_dim, self.theta = head_dim, theta
        weakref.finalize(self, lib.mi_rope_table_destroy, self._h)

    def cover(self, positions: int) -> None:
        _check(lib.mi_rope_table_cover(self._h, positions))

    def _info(self):
        n, data = C.c_int(), _vp()
        _check(lib.mi_rope_table_info(self._h, C.byref(n), C.byref(data)))
        return n.value, data.value

    def _data(self):
        return self._info()[1]

    @property
    def positions(self) -> int:
        return self._info()[0]

    @property
    def nbytes(self) -> int:
        return self.positions * self.head_dim * 4

    def to_numpy(self) -> np.ndarray:
        n, data = self._info()
        out = np.empty((n, self.head_dim // 2, 2), np.float32)
        if n:
            _d2h(out, data)
        return out


class Halves(enum.IntEnum):
    Both = 0
    Keys = 1
    Values = 2


class ImportanceScores:
    """The EWMA of each (layer, page)'s attention mass on the device
    (importance_scores.h:27-66)."""

    default_alpha = 0.2

    def __init__(self, layers: int, max_pages: int, alpha: float = 0.2):
        h = _vp()
        _check(lib.mi_scores_create(layers, max_pages, alpha, C.byref(h)))
        self._h = h.value
        weakref.finalize(self, lib.mi_scores_destroy, self._h)

    def _info(self):
        l, m, a, d = C.c_int(), C.c_int(), C.c_float(), C.c_size_t()
        _check(lib.mi_scores_info(self._h, C.byref(l), C.byref(m), C.byref(a), C.byref(d)))
        return l.value, m.value, a.value, d.value

    layers = property(lambda self: self._info()[0])
    max_pages = property(lambda self: self._info()[1])
    alpha = property(lambda self: self._info()[2])
    downloads = property(lambda self: self._info()[3])

    @property
    def nbytes(self) -> int:
        l, m, _, _ = self._info()
        return l * m * 4

    def row(self, layer: int) -> int:
        """The device address of a layer's scores, for a fused fold."""
        p = _vp()
        _check(lib.mi_scores_layer_row(self._h, layer, C.byref(p)))
        return p.value

    def fold(self, layer: int, mass: FloatTensor, heads: int, pages: int) -> None:
        if heads > 0 and pages > 0 and mass.numel < heads * pages:
            raise ValueError(f"the mass of {heads} heads over {pages} pages needs "
                             f"{heads * pages} floats; got {mass.numel}")
        _check(lib.mi_scores_fold(self._h, layer, mass.address, heads, pages))

    def download(self) -> np.ndarray:
        l, m, _, _ = self._info()
        out = np.empty((l, m), np.float32)
        _check(lib.mi_scores_download(self._h, out.ctypes.data, out.size))
        return out

    def upload(self, host) -> None:
        h = np.ascontiguousarray(host, np.float32)
        if h.ndim != 2:
            raise ValueError(f"scores to put back are (layers, max_pages); got {h.ndim} dimensions")
        _check(lib.mi_scores_upload(self._h, h.ctypes.data, h.shape[0], h.shape[1]))


class ShadowStore:
    """FP16 shadows in pinned host memory (shadow_store.h:23-85)."""

    allocation_bytes = 2 << 20

    def __init__(self, page_bytes: int):
        h = _vp()
        _check(lib.mi_shadows_create(page_bytes, C.byref(h)))
        self._h = h.value
        self.page_bytes = page_bytes
        weakref.finalize(self, lib.mi_shadows_destroy, self._h)

    def take(self, layer: int, page: int, tensor) -> None:
        span = _span(tensor)
        _need(span, self.page_bytes // 2, "a page's bytes")
        _check(lib.mi_shadows_take(self._h, layer, page, span.address))

    def contains(self, layer: int, page: int) -> bool:
        out = C.c_int()
        _check(lib.mi_shadows_contains(self._h, layer, page, C.byref(out)))
        return bool(out.value)

    def shadow(self, layer: int, page: int) -> np.ndarray:
        out = np.empty(self.page_bytes, np.uint8)
        _check(lib.mi_shadows_read(self._h, layer, page, out.ctypes.data, out.nbytes))
        return out

    @property
    def count(self) -> int:
        n = C.c_size_t()
        _check(lib.mi_shadows_count(self._h, C.byref(n)))
        return n.value

    @property
    def bytes(self) -> int:
        n = C.c_size_t()
        _check(lib.mi_shadows_bytes(self._h, C.byref(n)))
        return n.value


def _int_array(values) -> C.Array:
    flat = [int(v) for v in values]
    return (C.c_int * max(len(flat), 1))(*flat)


def _map_args(tier_map):
    rows = [list(map(int, row)) for row in (tier_map or [])]
    flat = [t for row in rows for t in row]
    return _int_array(flat), _int_array([len(r) for r in rows]), len(rows)


class PagedKVCache:
    """The per-tier VMM allocator (paged_kv_cache.h:112-227). No method
    returns a device address: pages move whenever a tier's tail retracts."""

    def __init__(self, page_bytes, capacity_pages):
        pb = (C.c_size_t * 4)(*[int(x) for x in page_bytes])
        cp = (C.c_size_t * 4)(*[int(x) for x in capacity_pages])
        h = _vp()
        _check(lib.mi_cache_create(pb, cp, C.byref(h)))
        self._h = h.value
        weakref.finalize(self, lib.mi_cache_destroy, self._h)

    def allocate(self, layer: int, page_index: int, tier) -> None:
        _check(lib.mi_cache_allocate(self._h, layer, page_index, _tier(tier)))

    def free(self, layer: int, page_index: int) -> None:
        _check(lib.mi_cache_free(self._h, layer, page_index))

    def free_pages(self, keys) -> None:
        keys = list(keys)
        _check(lib.mi_cache_free_pages(self._h, _int_array([x for k in keys for x in k]),
                                       len(keys)))

    def replace(self, key, staged) -> None:
        _check(lib.mi_cache_replace(self._h, key[0], key[1], staged[0], staged[1]))

    def replace_pages(self, pairs) -> None:
        pairs = list(pairs)
        flat = [x for key, staged in pairs for x in (*key, *staged)]
        _check(lib.mi_cache_replace_pages(self._h, _int_array(flat), len(pairs)))

    def write(self, layer: int, page_index: int, data) -> None:
        if not isinstance(data, np.ndarray) or not data.flags.c_contiguous:
            raise ValueError("a page is written from a C-contiguous array")
        _check(lib.mi_cache_write(self._h, layer, page_index, data.ctypes.data, data.nbytes))

    def read(self, layer: int, page_index: int) -> np.ndarray:
        tier, _ = self.locate(layer, page_index)
        out = np.empty(self.page_bytes(tier), np.uint8)
        _check(lib.mi_cache_read(self._h, layer, page_index, out.ctypes.data, out.nbytes))
        return out

    def locate(self, layer: int, page_index: int):
        t, s = C.c_int(), C.c_size_t()
        _check(lib.mi_cache_locate(self._h, layer, page_index, C.byref(t), C.byref(s)))
        return Tier(t.value), s.value

    def __contains__(self, key) -> bool:
        out = C.c_int()
        _check(lib.mi_cache_contains(self._h, key[0], key[1], C.byref(out)))
        return bool(out.value)

    def pages(self, tier) -> list:
        n = C.c_size_t()
        _check(lib.mi_cache_pages(self._h, _tier(tier), None, 0, C.byref(n)))
        buf = (C.c_int * max(2 * n.value, 1))()
        _check(lib.mi_cache_pages(self._h, _tier(tier), buf, n.value, C.byref(n)))
        return [(buf[2 * i], buf[2 * i + 1]) for i in range(n.value)]

    def _get(self, fn, tier) -> int:
        out = C.c_size_t()
        _check(fn(self._h, _tier(tier), C.byref(out)))
        return out.value

    def page_bytes(self, tier) -> int:
        return self._get(lib.mi_cache_page_bytes, tier)

    def reserved_bytes(self, tier) -> int:
        return self._get(lib.mi_cache_reserved_bytes, tier)

    def mapped_bytes(self, tier) -> int:
        return self._get(lib.mi_cache_mapped_bytes, tier)

    def keep_spare_granules(self, tier, granules: int) -> None:
        _check(lib.mi_cache_keep_spare_granules(self._h, _tier(tier), granules))

    def spare_granules(self, tier) -> int:
        return self._get(lib.mi_cache_spare_granules, tier)

    def drain_releases(self) -> None:
        """Waits until every granule the ranges gave up is unmapped and back
        with the driver (a thread of the cache's releases them after the call
        that gave them up returns)."""
        _check(lib.mi_cache_drain_releases(self._h))

    @property
    def granule_bytes(self) -> int:
        out = C.c_size_t()
        _check(lib.mi_cache_granule_bytes(self._h, C.byref(out)))
        return out.value


def fail_next_granules(n: int) -> None:
    """Test hook: the next n granule maps fail as out of memory."""
    _check(lib.mi_debug_fail_next_granules(n))


class KVPages:
    """The engine's KV cache on pages (kv_pages.h:105-412). Keeps its
    allocator alive."""

    def __init__(self, allocator: PagedKVCache, layers: int, page_tokens: int, kv_heads: int,
                 head_dim: int, tier, halves=Halves.Both, tier_map=None, always_seal=False):
        flat, lengths, rows = _map_args(tier_map)
        h = _vp()
        _check(lib.mi_kv_create(allocator._h, layers, page_tokens, kv_heads, head_dim,
                                _tier(tier), int(halves), flat if rows else None,
                                lengths if rows else None, rows, int(bool(always_seal)),
                                C.byref(h)))
        self._h = h.value
        self._allocator = allocator
        weakref.finalize(self, lib.mi_kv_destroy, self._h)

    @staticmethod
    def seals_for(tier, tier_map=None, always_seal=False) -> bool:
        flat, lengths, rows = _map_args(tier_map)
        out = C.c_int()
        _check(lib.mi_kv_seals_for(_tier(tier), flat if rows else None, lengths if rows else None,
                                   rows, int(bool(always_seal)), C.byref(out)))
        return bool(out.value)

    def _info(self) -> _KVInfo:
        info = _KVInfo()
        _check(lib.mi_kv_info_get(self._h, C.byref(info)))
        return info

    page_tokens = property(lambda self: self._info().page_tokens)
    pages_per_layer = property(lambda self: self._info().pages_per_layer)
    layers = property(lambda self: self._info().layers)
    capacity_tokens = property(lambda self: self._info().capacity_tokens)
    page_bytes = property(lambda self: self._info().page_bytes)
    kv_width = property(lambda self: self._info().kv_width)
    tier = property(lambda self: Tier(self._info().tier))
    halves = property(lambda self: Halves(self._info().halves))
    storage_tier = property(lambda self: Tier(self._info().storage_tier))
    seals = property(lambda self: bool(self._info().seals))
    born_at_one_tier = property(lambda self: bool(self._info().born_at_one_tier))
    shadow_count = property(lambda self: self._info().shadow_count)
    shadow_bytes = property(lambda self: self._info().shadow_bytes)

    def reserve(self, tokens: int) -> None:
        _check(lib.mi_kv_reserve(self._h, tokens))

    def store(self, layer: int, keys, values, start: int, n: int) -> None:
        _non_negative(n, "n")
        width = self.kv_width
        k = _need(_span(keys), n * width, "keys")
        v = _need(_span(values), n * width, "values")
        _check(lib.mi_kv_store(self._h, layer, k, v, start, n))

    def attention(self, layer: int, q, k_bias, rope, out, seq_q: int, seq_k: int, heads: int,
                  kv_heads: int, head_dim: int, keys=None, values=None, mass=None, partials=None,
                  scores=None):
        """`scores`, beyond the reference's surface, is an ImportanceScores
        whose row for `layer` the step's mass is folded into in the same
        launch sequence."""
        if seq_q > seq_k:
            raise ValueError(f"seq_q {seq_q} exceeds seq_k {seq_k}")
        _non_negative(seq_q, "seq_q")
        qa = _need(_span(q), seq_q * heads * head_dim, "q")
        oa = _need(_span(out), seq_q * heads * head_dim, "out")
        ba = _need(_span(k_bias), kv_heads * head_dim, "k_bias") if k_bias is not None else None
        ka = _need(_span(keys), seq_q * kv_heads * head_dim, "keys") if keys is not None else None
        va = (_need(_span(values), seq_q * kv_heads * head_dim, "values")
              if values is not None else None)
        P = self.page_tokens
        pages = -(-seq_k // P)
        ma = None
        if mass is not None:
            if mass.numel < pages * heads:
                raise ValueError(f"the per-page attention mass needs {pages * heads} floats, "
                                 f"(heads, pages); got {mass.numel}")
            ma = mass.address
        sa, alpha = None, 0.0
        if scores is not None:
            sa, alpha = scores.row(layer), scores.alpha
            if pages > scores.max_pages:
                raise ValueError(f"{pages} pages; the scores hold up to {scores.max_pages}")
        pa = _floats(partials, _attention_partials(head_dim), "attention's partials")
        _check(lib.mi_kv_attention(self._h, layer, qa, ba, rope._h if rope is not None else None,
                                   oa, seq_q, seq_k, heads, kv_heads, head_dim, ka, va, ma, sa,
                                   alpha, pa))

    def attention_layers(self, first_layer: int, layers: int, q, out, seq_k: int, heads: int,
                         kv_heads: int, head_dim: int, keys=None, values=None, mass=None,
                         scores=None):
        """Beyond the reference's surface: one decode query per head for
        `layers` consecutive layers in one launch. q and out hold (layers,
        heads, head_dim) fp16, keys/values (layers, kv_width) (the query's
        own rows), mass (layers, heads, pages) floats; `scores` an
        ImportanceScores whose rows first_layer.. take the fold. Each layer's
        results are attention(layer, ..., seq_q=1)'s within the attention
        tolerance (the streamed launch splits the pages differently)."""
        _non_negative(layers, "layers")
        per_q = heads * head_dim
        width = kv_heads * head_dim
        qa = _need(_span(q), layers * per_q, "q")
        oa = _need(_span(out), layers * per_q, "out")
        ka = _need(_span(keys), layers * width, "keys") if keys is not None else None
        va = _need(_span(values), layers * width, "values") if values is not None else None
        pages = -(-seq_k // self.page_tokens)
        ma = None
        if mass is not None:
            if mass.numel < layers * heads * pages:
                raise ValueError(f"the per-page attention mass of {layers} layers needs "
                                 f"{layers * heads * pages} floats; got {mass.numel}")
            ma = mass.address
        sa, stride, alpha = None, 0, 0.0
        if scores is not None:
            if pages > scores.max_pages:
                raise ValueError(f"{pages} pages; the scores hold up to {scores.max_pages}")
            sa, stride, alpha = scores.row(first_layer), scores.max_pages, scores.alpha
        _check(lib.mi_kv_attention_layers(self._h, first_layer, layers, qa, per_q, oa, per_q,
                                          seq_k, heads, kv_heads, head_dim, ka, va, width, ma,
                                          heads * pages, sa, stride, alpha))

    def attention_kept(self, layer: int, q, k_bias, rope, out, seq_k: int, heads: int,
                       kv_heads: int, head_dim: int, keys=None, values=None) -> None:
        """Beyond the reference's surface: one layer's decode (one query a
        head) keeping its page statistics for fold_kept, which forms every
        layer's masses and folds them into the scores in one launch."""
        per_q = heads * head_dim
        width = kv_heads * head_dim
        qa = _need(_span(q), per_q, "q")
        oa = _need(_span(out), per_q, "out")
        ba = _need(_span(k_bias), width, "k_bias") if k_bias is not None else None
        ka = _need(_span(keys), width, "keys") if keys is not None else None
        va = _need(_span(values), width, "values") if values is not None else None
        _check(lib.mi_kv_attention_kept(self._h, layer, qa, ba, rope._h if rope else None, oa,
                                        seq_k, heads, kv_heads, head_dim, ka, va))

    def store_at(self, layer: int, keys, values, position: DeviceIndex) -> None:
        """Beyond the reference's surface: one row stored at the position
        held in device memory (`position`, one int), read when the kernel
        runs; the row that completes a page seals it."""
        width = self.kv_width
        _check(lib.mi_kv_store_at(self._h, layer, _need(_span(keys), width, "keys"),
                                  _need(_span(values), width, "values"), position.address))

    def attention_at(self, layer: int, q, k_bias, rope, out, seq_k: DeviceIndex, max_seq_k: int,
                     heads: int, kv_heads: int, head_dim: int, keys, values) -> None:
        """Beyond the reference's surface: one layer's decode at the seq_k
        held in device memory, the launch sized for max_seq_k; to the bit
        attention(..., partials) at that seq_k."""
        per_q = heads * head_dim
        width = kv_heads * head_dim
        ba = _need(_span(k_bias), width, "k_bias") if k_bias is not None else None
        _check(lib.mi_kv_attention_at(self._h, layer, _need(_span(q), per_q, "q"), ba,
                                      rope._h if rope else None, _need(_span(out), per_q, "out"),
                                      seq_k.address, max_seq_k, heads, kv_heads, head_dim,
                                      _need(_span(keys), width, "keys"),
                                      _need(_span(values), width, "values")))

    def rope_store(self, layer: int, qk, qk_out, q_heads: int, position: DeviceIndex,
                   rope: "RopeTable", values, norm=None) -> None:
        """Beyond the reference's surface, for a cache that does not seal: a
        decode row's RoPE and store in one launch. qk holds q_heads then
        kv_heads rows of head_dim; they are rotated into qk_out at the
        position held in device memory (rope's angles), and the rotated k
        rows and `values` are stored there. norm = (x, weight, out, eps)
        adds the RMSNorm of the fp32 row x to the same launch. The bits of
        rmsnorm_f32, rope_from_table and store."""
        width = self.kv_width
        rows = q_heads * rope.head_dim + width
        qa = _need(_span(qk), rows, "qk")
        oa = _need(_span(qk_out), rows, "qk_out")
        if qa == oa:
            raise ValueError("rope cannot write over its input")
        if position.count < 1:
            raise ValueError("the position holds no value")
        xa = wa = na = None
        hidden, eps = 0, 0.0
        if norm is not None:
            x, weight, out, eps = norm
            hidden = x.numel
            xa = x.address
            wa = _need(_span(weight), hidden, "norm weight")
            na = _need(_span(out), hidden, "normed")
        _check(lib.mi_kv_rope_store(self._h, layer, qa, oa, q_heads, position.address, rope._h,
                                    _need(_span(values), width, "values"), xa, wa, na, hidden,
                                    float(eps)))

    def attend_row(self, layer: int, qk, qk_out, q_heads: int, seq_k: int, rope: "RopeTable",
                   values, out, norm=None) -> None:
        """Beyond the reference's surface, for a cache that does not seal:
        rope_store at position seq_k - 1 then attention's one-query split
        decode over the positions before seq_k, as two launches (the pages
        launch turns q and the row's k, stores the row and forms the
        RMSNorm; then the combine). qk_out, when not None, receives the
        turned rows. The bits of rope_store then attention with partials."""
        width = self.kv_width
        hd = rope.head_dim
        rows = q_heads * hd + width
        qa = _need(_span(qk), rows, "qk")
        oa = _need(_span(qk_out), rows, "qk_out") if qk_out is not None else None
        if qa == oa:
            raise ValueError("rope cannot write over its input")
        xa = wa = na = None
        hidden, eps = 0, 0.0
        if norm is not None:
            x, weight, normed, eps = norm
            hidden = x.numel
            xa = x.address
            wa = _need(_span(weight), hidden, "norm weight")
            na = _need(_span(normed), hidden, "normed")
        _check(lib.mi_kv_attend_row(self._h, layer, qa, oa, q_heads, seq_k, rope._h,
                                    _need(_span(values), width, "values"),
                                    _need(_span(out), q_heads * hd, "out"), xa, wa, na, hidden,
                                    float(eps)))

    def stored_on_device(self, end: int) -> None:
        """Records that the positions before `end` were stored by store_at."""
        _check(lib.mi_kv_stored_on_device(self._h, end))

    def fold_kept(self, scores=None, mass=None, seq_k: int | None = None, heads: int = 0) -> None:
        """Every layer's page masses (mass: (layers, heads, pages) floats,
        if given) and their fold into `scores` (an ImportanceScores, if
        given), for the step every layer was attended in by attention_kept."""
        ma, mstride = None, 0
        if mass is not None:
            if seq_k is None or heads <= 0:
                raise ValueError("a mass output needs the step's seq_k and heads")
            pages = -(-seq_k // self.page_tokens)
            if mass.numel < self.layers * heads * pages:
                raise ValueError(f"the per-page attention mass of {self.layers} layers needs "
                                 f"{self.layers * heads * pages} floats; got {mass.numel}")
            ma, mstride = mass.address, heads * pages
        sa, sstride, alpha = None, 0, 0.0
        if scores is not None:
            sa, sstride, alpha = scores.row(0), scores.max_pages, scores.alpha
        _check(lib.mi_kv_fold_kept(self._h, ma, mstride, sa, sstride, alpha))

    def page_tier(self, layer: int, page: int) -> Tier:
        t = C.c_int()
        _check(lib.mi_kv_page_tier(self._h, layer, page, C.byref(t)))
        return Tier(t.value)

    def has_shadow(self, layer: int, page: int) -> bool:
        out = C.c_int()
        _check(lib.mi_kv_has_shadow(self._h, layer, page, C.byref(out)))
        return bool(out.value)

    def shadow(self, layer: int, page: int) -> np.ndarray:
        n = page_bytes(self.page_tokens, self.kv_width)
        out = np.empty(n, np.uint8)
        _check(lib.mi_kv_shadow(self._h, layer, page, out.ctypes.data, n))
        return out

    def _per_page(self, dtype, fill):
        info = self._info()
        out = np.zeros((info.layers, info.pages_per_layer), dtype)
        if out.size:
            _check(fill(out))
        return out

    def page_tiers(self) -> np.ndarray:
        return self._per_page(np.int8, lambda o: lib.mi_kv_page_tiers(self._h, o.ctypes.data,
                                                                       o.size))

    def shadowed(self) -> np.ndarray:
        return self._per_page(np.uint8, lambda o: lib.mi_kv_flags(self._h, 0, o.ctypes.data,
                                                                   o.size)).astype(bool)

    def evicted(self) -> np.ndarray:
        return self._per_page(np.uint8, lambda o: lib.mi_kv_flags(self._h, 1, o.ctypes.data,
                                                                   o.size)).astype(bool)

    def downgrade(self, layer: int, page: int, target) -> None:
        _check(lib.mi_kv_downgrade(self._h, layer, page, _tier(target)))

    def upgrade(self, layer: int, page: int, target) -> None:
        _check(lib.mi_kv_upgrade(self._h, layer, page, _tier(target)))

    def move_pages(self, moves) -> None:
        """`moves`: (layer, page, tier) triples, a list or an (n, 3) array."""
        flat = np.ascontiguousarray(np.asarray(moves, dtype=np.int64).reshape(-1, 3),
                                    dtype=np.int32)
        bad = (flat[:, 2] < 0) | (flat[:, 2] > 3)
        if bad.any():
            raise ValueError(f"tier {int(flat[bad][0, 2])} is not one of the four")
        _check(lib.mi_kv_move_pages(self._h, flat.ctypes.data_as(_ip), len(flat)))

    def pin_shadows(self, pages: int) -> None:
        """Pins host memory for `pages` more FP16 shadows now (beyond the
        reference: its shadows are pinned as they are taken)."""
        _check(lib.mi_kv_pin_shadows(self._h, pages))

    def evict(self, layer: int, page: int) -> None:
        _check(lib.mi_kv_evict(self._h, layer, page))

    def mask(self, layer: int, page: int) -> None:
        _check(lib.mi_kv_mask(self._h, layer, page))

    def birth_tier(self, layer: int, page: int) -> Tier:
        t = C.c_int()
        _check(lib.mi_kv_birth_tier(self._h, layer, page, C.byref(t)))
        return Tier(t.value)

    @property
    def last_move(self):
        has, ints = C.c_int(), (C.c_int * 4)()
        nbytes, secs = (C.c_size_t * 2)(), (C.c_double * 2)()
        _check(lib.mi_kv_last_move(self._h, C.byref(has), ints, nbytes, secs))
        if not has.value:
            return None
        return {"layer": ints[0], "page": ints[1], "from_tier": Tier(ints[2]),
                "to_tier": Tier(ints[3]), "from_bytes": nbytes[0], "to_bytes": nbytes[1],
                "seconds": secs[0], "shadow_seconds": secs[1]}

    @property
    def last_batch(self):
        has, moves, shadows, secs = C.c_int(), C.c_size_t(), C.c_size_t(), C.c_double()
        _check(lib.mi_kv_last_batch(self._h, C.byref(has), C.byref(moves), C.byref(shadows),
                                    C.byref(secs)))
        if not has.value:
            return None
        phases = (C.c_double * 3)()
        _check(lib.mi_kv_last_batch_phases(self._h, phases))
        return {"moves": moves.value, "shadows_taken": shadows.value, "seconds": secs.value,
                "prepare_seconds": phases[0], "allocate_seconds": phases[1],
                "finish_seconds": phases[2]}


def page_bytes(page_tokens: int, kv_width: int) -> int:
    """Bytes in one FP16 page: P rows of keys then P of values."""
    return int(lib.mi_fp16_page_bytes(page_tokens, kv_width))


def _device_attention(q, k, v, k_bias, rope_table, out, seq_q, seq_k, heads, kv_heads, head_dim,
                      partials=None):
    if seq_q > seq_k:
        raise ValueError(f"seq_q {seq_q} exceeds seq_k {seq_k}")
    qa = _need(_span(q), seq_q * heads * head_dim, "q")
    ka = _need(_span(k), seq_k * kv_heads * head_dim, "k")
    va = _need(_span(v), seq_k * kv_heads * head_dim, "v")
    ba = _need(_span(k_bias), kv_heads * head_dim, "k_bias") if k_bias is not None else None
    oa = _need(_span(out), seq_q * heads * head_dim, "out")
    pa = _floats(partials, _attention_partials(head_dim), "attention's partials")
    data = rope_table._data() if rope_table is not None else None
    positions = rope_table.positions if rope_table is not None else 0
    if ba is not None and (rope_table is None or positions < seq_k):
        raise ValueError(f"a key bias needs a RoPE table for head_dim {head_dim} covering "
                         f"{seq_k} positions")
    _check(lib.mi_attention(qa, ka, va, ba, data, positions, oa, seq_q, seq_k, heads, kv_heads,
                            head_dim, pa, None))


def _device_rmsnorm(x, weight, out, rows, hidden, eps):
    xa = _need(_span(x), rows * hidden, "x")
    wa = _need(_span(weight), hidden, "weight")
    oa = _need(_span(out), rows * hidden, "out")
    _check(lib.mi_rmsnorm(xa, 0, wa, oa, rows, hidden, eps, None))


def _device_rmsnorm_f32(x: FloatTensor, weight, out, rows, hidden, eps):
    if x.numel < rows * hidden:
        raise ValueError(f"x holds {x.numel}, and the operation needs {rows * hidden}")
    wa = _need(_span(weight), hidden, "weight")
    oa = _need(_span(out), rows * hidden, "out")
    _check(lib.mi_rmsnorm(x.address, 1, wa, oa, rows, hidden, eps, None))


def _device_rope(x, positions: DeviceIndex, out, seq, heads, head_dim, theta):
    xa = _need(_span(x), seq * heads * head_dim, "x")
    if positions.count < seq:
        raise ValueError(f"positions holds {positions.count}, and the operation needs {seq}")
    oa = _need(_span(out), seq * heads * head_dim, "out")
    if xa == oa:
        raise ValueError("rope cannot write over its input")
    _check(lib.mi_rope(xa, positions.address, oa, seq, heads, head_dim, theta, None))


def _device_rope_from_table(x, positions: DeviceIndex, table: "RopeTable", out, seq, heads,
                            head_dim):
    """_device_rope's rows with the angles read from `table` (beyond the
    reference): every position must be below table.positions."""
    xa = _need(_span(x), seq * heads * head_dim, "x")
    if positions.count < seq:
        raise ValueError(f"positions holds {positions.count}, and the operation needs {seq}")
    oa = _need(_span(out), seq * heads * head_dim, "out")
    if xa == oa:
        raise ValueError("rope cannot write over its input")
    if table.head_dim != head_dim:
        raise ValueError(f"the table is for head_dim {table.head_dim}, not {head_dim}")
    covered, data = table._info()
    _check(lib.mi_rope_from_table(xa, positions.address, data, covered, oa, seq, heads, head_dim,
                                  None))


def _device_swiglu(gate, up, out, count):
    ga = _need(_span(gate), count, "gate")
    ua = _need(_span(up), count, "up")
    oa = _need(_span(out), count, "out")
    if oa in (ga, ua):
        raise ValueError("swiglu cannot write over its input")
    _check(lib.mi_swiglu(ga, ua, oa, count, None))


def _device_add(a, b, out, count):
    _check(lib.mi_add(_need(_span(a), count, "a"), _need(_span(b), count, "b"),
                      _need(_span(out), count, "out"), count, None))


def _device_copy(source, target, count):
    sa = _need(_span(source), count, "source")
    ta = _need(_span(target), count, "target")
    _check(lib.mi_memcpy(ta, sa, 2 * count, 2))


def _device_linear(x, weight, bias, out, rows, in_features, out_features):
    xa = _need(_span(x), rows * in_features, "x")
    wa = _need(_span(weight), out_features * in_features, "weight")
    ba = _need(_span(bias), out_features, "bias") if bias is not None else None
    oa = _need(_span(out), rows * out_features, "out")
    _check(lib.mi_linear(xa, wa, ba, oa, rows, in_features, out_features, None))


def _device_linear_accumulate(x, weight, out: FloatTensor, rows, in_features, out_features):
    """out += x @ weight.T in fp32: a projection added into the residual
    stream with no fp16 rounding (bindings_device.cpp:351-365)."""
    xa = _need(_span(x), rows * in_features, "x")
    wa = _need(_span(weight), out_features * in_features, "weight")
    oa = _floats(out, rows * out_features, "out")
    _check(lib.mi_linear_f32(xa, wa, oa, 1, rows, in_features, out_features, None))


def _device_embed(ids: DeviceIndex, table, out, hidden, vocab):
    ta = _need(_span(table), vocab * hidden, "table")
    oa = _need(_span(out), ids.count * hidden, "out")
    _check(lib.mi_embed(ids.address, ids.count, ta, oa, 0, hidden, vocab, None))


def _device_embed_f32(ids: DeviceIndex, table, out: FloatTensor, hidden, vocab):
    """The embedding gather, widened exactly to fp32 (bindings_device.cpp:321-334)."""
    ta = _need(_span(table), vocab * hidden, "table")
    oa = _floats(out, ids.count * hidden, "out")
    _check(lib.mi_embed(ids.address, ids.count, ta, oa, 1, hidden, vocab, None))


def scratch_elements(rows: int, vocab: int) -> int:
    """fp16 elements of scratch that logits or greedy need for `rows` rows."""
    out = C.c_size_t()
    _check(lib.mi_scratch_elements(rows, vocab, C.byref(out)))
    return out.value


def _logits_args(x, head, scratch, first_row, rows, hidden, vocab):
    _non_negative(first_row, "first_row")
    _non_negative(rows, "rows")
    xa = _need(_span(x), (first_row + rows) * hidden, "x")
    ha = _need(_span(head), vocab * hidden, "head")
    sp = _span(scratch)
    sa = _need(sp, scratch_elements(rows, vocab), "scratch")
    return xa, ha, sa, sp.count


def logits(x, head, scratch, first_row: int, rows: int, hidden: int, vocab: int) -> np.ndarray:
    """fp32 logits for rows [first_row, first_row + rows) of x, to the host
    (bindings_device.cpp:133-157)."""
    xa, ha, sa, held = _logits_args(x, head, scratch, first_row, rows, hidden, vocab)
    out = np.empty((rows, vocab), np.float32)
    _check(lib.mi_logits(xa, ha, sa, held, first_row, rows, hidden, vocab, out.ctypes.data))
    return out


def greedy(x, head, scratch, first_row: int, rows: int, hidden: int, vocab: int) -> np.ndarray:
    """The argmax token of each row's logits, computed on the device
    (bindings_device.cpp:161-195); a row with no finite logit raises."""
    xa, ha, sa, held = _logits_args(x, head, scratch, first_row, rows, hidden, vocab)
    out = np.empty(rows, np.int32)
    _check(lib.mi_greedy(xa, ha, sa, held, first_row, rows, hidden, vocab, out.ctypes.data))
    return out


def _upload_f32(host) -> FloatTensor:
    h = np.ascontiguousarray(host, np.float32).reshape(-1)
    t = FloatTensor(h.size)
    _h2d(t.address, h)
    return t


def random_half(tensor, seed: int, scale: float) -> None:
    """Fill a device fp16 tensor with synthetic values, uniform in
    [-scale, scale), made on the device from `seed`."""
    sp = _span(tensor)
    _check(lib.mi_random_half(sp.address, sp.count, seed, scale))


class DecodeStep:
    """A whole decode step of a Qwen2 / Llama-shaped decoder as one HIP
    graph (beyond the reference, whose host sequences the step a call at a
    time: model.py:332-403, engine.py:1180-1206). `shape` has layers,
    hidden, intermediate, heads, kv_heads, head_dim, vocab, rms_eps and
    rope_theta; `layers` is a list of dicts of fp16 device tensors named as
    _LAYER_TENSORS (biases may be None). The cache must seal its pages."""

    def __init__(self, cache: KVPages, shape: dict, embed, final_norm, head, layers,
                 scores: ImportanceScores | None = None, score_every: int = 1):
        sh = _ModelShape(**{f: shape[f] for f, _ in _ModelShape._fields_})
        arr = (_LayerWeights * len(layers))()
        for i, tensors in enumerate(layers):
            for name in _LAYER_TENSORS:
                t = tensors.get(name)
                setattr(arr[i], name, _span(t).address if t is not None else None)
        h = _vp()
        _check(lib.mi_decode_step_create(C.byref(h), cache._h, C.byref(sh), _span(embed).address,
                                         _span(final_norm).address, _span(head).address, arr,
                                         scores._h if scores is not None else None, score_every))
        self._h = h.value
        # The step reads these while it lives.
        self._keep = (cache, scores, embed, final_norm, head, layers)
        self.vocab = shape["vocab"]
        weakref.finalize(self, lib.mi_decode_step_destroy, self._h)

    def run(self, token: int, position: int, steps: int, graphed: bool = True):
        """`steps` greedy steps from `position`, feeding `token` first:
        (tokens chosen, device milliseconds of the replays). graphed=False
        makes the same launches from the host a step at a time."""
        out = np.empty(steps, np.int32)
        ms = C.c_double()
        fn = lib.mi_decode_step_run if graphed else lib.mi_decode_step_run_eager
        _check(fn(self._h, token, position, steps, out.ctypes.data_as(C.POINTER(C.c_int32)),
                  C.byref(ms)))
        return out, ms.value

    def prefill(self, tokens, position: int = 0, chunk: int = 2048):
        """The prompt at positions [position, position + len(tokens)) in
        chunks of `chunk` rows: (the first decode token, device
        milliseconds). The logits after the last row are logits()."""
        ids = np.ascontiguousarray(tokens, np.int32).reshape(-1)
        first = C.c_int32()
        ms = C.c_double()
        _check(lib.mi_decode_step_prefill(self._h, ids.ctypes.data_as(C.POINTER(C.c_int32)),
                                          ids.size, position, chunk, C.byref(first),
                                          C.byref(ms)))
        return first.value, ms.value

    def logits(self) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        _check(lib.mi_decode_step_logits(self._h, out.ctypes.data_as(_fp), out.size))
        return out

    @property
    def launches(self) -> int:
        n = C.c_int()
        _check(lib.mi_decode_step_launches(self._h, C.byref(n)))
        return n.value

    #: The GEMVs projection_plans() names, in its order.
    PLAN_NAMES = ("output", "gate_up", "down", "head")

    def projection_plans(self) -> dict:
        """The plans the last step's GEMVs ran as (beyond the reference):
        {name: {rows, in, split, pipelined, waves, blocks}} for layer 0's
        output, gate/up and down projections and the head. `split` is the
        waves a row is split over; `pipelined` that the grid was the
        device's resident one, each wave taking several rows."""
        count = C.c_size_t()
        _check(lib.mi_decode_step_plans(self._h, None, 0, C.byref(count)))
        ints = np.zeros(count.value, np.int32)
        _check(lib.mi_decode_step_plans(self._h, ints.ctypes.data_as(_ip), ints.size,
                                        C.byref(count)))
        plans = {}
        for row in ints.reshape(-1, 7):
            what, rows, n_in, split, pipelined, waves, blocks = (int(x) for x in row)
            plans[self.PLAN_NAMES[what]] = dict(rows=rows, n_in=n_in, split=split,
                                                pipelined=bool(pipelined), waves=waves,
                                                blocks=blocks)
        return plans


device = SimpleNamespace(
    Span=Span,
    view=lambda tensor, offset, count: Span(tensor, offset, count),
    empty=lambda count: DeviceTensor(count),
    empty_f32=lambda count: FloatTensor(count),
    FloatTensor=FloatTensor,
    upload_f32=_upload_f32,
    index=DeviceIndex,
    DeviceIndex=DeviceIndex,
    embed=_device_embed,
    embed_f32=_device_embed_f32,
    linear=_device_linear,
    linear_accumulate=_device_linear_accumulate,
    rmsnorm=_device_rmsnorm,
    rmsnorm_f32=_device_rmsnorm_f32,
    rope=_device_rope,
    rope_from_table=_device_rope_from_table,
    attention=_device_attention,
    attention_partials=_attention_partials,
    attention_split=lambda seq_q, seq_k, heads, kv_heads, page_tokens=0: _split(
        seq_q, seq_k, heads, kv_heads, page_tokens),
    RopeTable=RopeTable,
    add=_device_add,
    swiglu=_device_swiglu,
    copy=_device_copy,
    page_tokens=P_DEFAULT,
    Halves=Halves,
    ImportanceScores=ImportanceScores,
    ShadowStore=ShadowStore,
    KVPages=KVPages,
    DecodeStep=DecodeStep,
    random_half=random_half,
    open_pages=(-1, -2),
    staging_page=-3,
    shadow_upload_page=-4,
    evicted_tier=4,
    page_bytes=page_bytes,
    scratch_elements=scratch_elements,
    logits=logits,
    greedy=greedy,
    synchronize=synchronize,
)


def _split(seq_q, seq_k, heads, kv_heads, page_tokens=0):
    s, k = C.c_int(), C.c_int()
    _check(lib.mi_attention_split(seq_q, seq_k, heads, kv_heads, page_tokens, C.byref(s),
                                  C.byref(k)))
    return s.value, k.value


class Stream:
    """A HIP stream of the default priority, ordered with the null stream."""

    def __init__(self):
        h = _vp()
        _check(lib.mi_stream_create(C.byref(h)))
        self.handle = h.value
        weakref.finalize(self, lib.mi_stream_destroy, self.handle)

    def synchronize(self) -> None:
        _check(lib.mi_stream_synchronize(self.handle))


def set_stream(stream: "Stream | None") -> None:
    """The stream the runtime objects launch on from this thread."""
    _check(lib.mi_set_stream(stream.handle if stream is not None else None))


class Graph:
    """The launches made on `stream` inside `with graph.capture():`,
    replayed by launch(). Every address the captured launches read is fixed
    at capture, so nothing may be allocated, freed or re-resolved between
    replays."""

    def __init__(self, stream: Stream):
        self.stream = stream
        self.exec = None

    def capture(self):
        graph = self

        class _Capture:
            def __enter__(self):
                set_stream(graph.stream)
                _check(lib.mi_graph_begin(graph.stream.handle))
                return graph

            def __exit__(self, *exc):
                e = _vp()
                status = lib.mi_graph_end(graph.stream.handle, C.byref(e))
                set_stream(None)
                if exc[0] is None:
                    _check(status)
                    graph.exec = e.value
                    weakref.finalize(graph, lib.mi_graph_destroy, graph.exec)
                return False

        return _Capture()

    def launch(self) -> None:
        _check(lib.mi_graph_launch(self.exec, self.stream.handle))


class Timer:
    """hipEvents on a stream (default: the null stream, which the library's
    kernels run on unless set_stream names another): elapsed milliseconds
    between start() and stop()."""

    def __init__(self, stream: "Stream | None" = None):
        self._stream = stream.handle if stream is not None else None
        a, b = _vp(), _vp()
        _check(lib.mi_event_create(C.byref(a)))
        _check(lib.mi_event_create(C.byref(b)))
        self._a, self._b = a.value, b.value
        weakref.finalize(self, lambda x, y: (lib.mi_event_destroy(x), lib.mi_event_destroy(y)),
                         self._a, self._b)

    def start(self) -> None:
        _check(lib.mi_event_record(self._a, self._stream))

    def stop(self) -> None:
        _check(lib.mi_event_record(self._b, self._stream))

    def elapsed_ms(self) -> float:
        ms = C.c_float()
        _check(lib.mi_event_elapsed_ms(self._a, self._b, C.byref(ms)))
        return ms.value


def library_path() -> str:
    return os.fspath(_LIB_PATH)
