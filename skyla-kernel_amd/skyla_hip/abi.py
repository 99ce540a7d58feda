"""ctypes binding of include/skyla_hip.h, shaped like the reference's `gpu` module.

The names and argument meanings are those of skyla-vk / skyla-metal as skyla-engine uses
them (Context::new, alloc_host, create_pipeline_sets, bind_set_buffers, record with a
Recorder, replay, marks, time_dispatch; skyla-vk/src/*.rs).  Errors raise SkylaHipError,
the counterpart of the anyhow::Error those methods return.

The library is loaded from skyla-kernel_amd/lib/libskyla_hip.so (or $SKYLA_HIP_LIB).  There
is no fallback: if the library or a device is missing, the calls fail loudly.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Callable, Sequence

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("SKYLA_HIP_LIB", os.path.join(_PKG, "lib", "libskyla_hip.so"))

OK, E_ARG, E_DEVICE, E_NO_KERNEL, E_OOM, E_STATE = 0, -1, -2, -3, -4, -5

_u32p = C.POINTER(C.c_uint32)
_vp = C.c_void_p

# (name, restype, argtypes) for every entry point declared in include/skyla_hip.h
SIGNATURES = [
    ("skyla_hip_last_error", C.c_char_p, []),
    ("skyla_hip_context_new", C.c_int, [C.c_int, C.POINTER(_vp)]),
    ("skyla_hip_context_free", None, [_vp]),
    ("skyla_hip_subgroup_size", C.c_uint32, [_vp]),
    ("skyla_hip_max_buffer", C.c_uint64, [_vp]),
    ("skyla_hip_device_name", C.c_int, [_vp, C.c_char_p, C.c_size_t]),
    ("skyla_hip_alloc", C.c_int, [_vp, C.c_uint64, C.POINTER(_vp)]),
    ("skyla_hip_buffer_free", None, [_vp]),
    ("skyla_hip_buffer_size", C.c_uint64, [_vp]),
    ("skyla_hip_buffer_host", _vp, [_vp]),
    ("skyla_hip_buffer_upload", C.c_int, [_vp, C.c_uint64, C.c_uint64]),
    ("skyla_hip_buffer_download", C.c_int, [_vp, C.c_uint64, C.c_uint64]),
    ("skyla_hip_buffer_device", _vp, [_vp]),
    ("skyla_hip_buffer_copy", C.c_int, [_vp, C.c_uint64, _vp, C.c_uint64, C.c_uint64]),
    ("skyla_hip_pipeline_new", C.c_int,
     [_vp, C.c_char_p, C.c_uint32, C.c_uint32, _u32p, C.c_uint32, C.c_uint32, C.POINTER(_vp)]),
    ("skyla_hip_pipeline_free", None, [_vp]),
    ("skyla_hip_pipeline_bind", C.c_int, [_vp, C.c_uint32, C.POINTER(_vp), C.c_uint32]),
    ("skyla_hip_pipeline_threads", C.c_int, [_vp, _u32p]),
    ("skyla_hip_record_begin", C.c_int, [_vp, C.c_int, C.POINTER(_vp)]),
    ("skyla_hip_record_dispatch", C.c_int, [_vp, _vp, C.c_uint32, _u32p, _u32p, C.c_uint32]),
    ("skyla_hip_record_barrier", C.c_int, [_vp]),
    ("skyla_hip_record_host_barrier", C.c_int, [_vp]),
    ("skyla_hip_record_mark", C.c_int, [_vp, C.c_char_p]),
    ("skyla_hip_record_end", C.c_int, [_vp, C.POINTER(_vp)]),
    ("skyla_hip_recording_free", None, [_vp]),
    ("skyla_hip_recording_len", C.c_uint32, [_vp]),
    ("skyla_hip_recording_launches", C.c_uint32, [_vp]),
    ("skyla_hip_replay", C.c_int, [_vp, _vp]),
    ("skyla_hip_replay_timed", C.c_int, [_vp, _vp, C.POINTER(C.c_double)]),
    ("skyla_hip_marks", C.c_int,
     [_vp, _vp, C.POINTER(C.c_char_p), C.POINTER(C.c_double), C.c_uint32, _u32p]),
    ("skyla_hip_time_dispatch", C.c_int,
     [_vp, _vp, _u32p, _u32p, C.c_uint32, C.c_uint32, C.POINTER(C.c_double)]),
    ("skyla_hip_dispatch_noalloc", C.c_int, [_vp, _vp, _u32p, _u32p, C.c_uint32]),
]

_lib = None


def tactic(key: str, default: str) -> str:
    """The value of tactic `key` from SKYLA_HIP_TACTIC ("key=value,key=value"; the last entry
    for a key wins), else `default`.  The runtime reads its own kernel-selection keys from the
    same variable; the engine reads its recording choices here."""
    value = default
    for item in os.environ.get("SKYLA_HIP_TACTIC", "").split(","):
        k, sep, v = item.partition("=")
        if sep and k.strip() == key:
            value = v.strip()
    return value


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Loads the C-ABI library and declares every signature (raises if any is missing)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise SkylaHipError(E_DEVICE, f"{path} is not built (run skyla-kernel_amd/build.py)")
    lib = C.CDLL(path)
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class SkylaHipError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


def _check(status: int) -> None:
    if status != OK:
        msg = _lib.skyla_hip_last_error().decode(errors="replace") if _lib else ""
        raise SkylaHipError(status, msg)


def _u32s(words: Sequence[int]):
    arr = (C.c_uint32 * max(1, len(words)))()
    for i, w in enumerate(words):
        arr[i] = int(w) & 0xFFFFFFFF
    return arr


class Buffer:
    """skyla-vk Buffer: HBM plus a host mirror (as_mut_slice / as_f32 / as_u32_mut)."""

    def __init__(self, ctx: "Context", handle: int, size: int):
        self.ctx, self._h, self.size = ctx, handle, size

    @property
    def handle(self) -> int:
        return self._h

    def host(self):
        """The host mirror as a numpy uint8 array (no copy)."""
        import numpy as np

        p = _lib.skyla_hip_buffer_host(self._h)
        if not p:
            _check(E_OOM)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), shape=(self.size,))

    def as_f32(self):
        return self.host().view("<f4")

    def as_u32(self):
        return self.host().view("<u4")

    def upload(self, off: int = 0, length: int | None = None) -> None:
        _check(_lib.skyla_hip_buffer_upload(self._h, off, self.size - off if length is None else length))

    def download(self, off: int = 0, length: int | None = None) -> None:
        _check(_lib.skyla_hip_buffer_download(self._h, off, self.size - off if length is None else length))

    def device_ptr(self) -> int:
        return _lib.skyla_hip_buffer_device(self._h)

    def copy_from(self, dst_off: int, src: "Buffer", src_off: int, length: int) -> None:
        _check(_lib.skyla_hip_buffer_copy(self._h, dst_off, src._h, src_off, length))

    def free(self) -> None:
        if self._h:
            _lib.skyla_hip_buffer_free(self._h)
            self._h = None


class Pipeline:
    def __init__(self, ctx: "Context", handle: int, name: str, spec: Sequence[int]):
        self.ctx, self._h, self.name, self.spec = ctx, handle, name, list(spec)

    def bind_buffers(self, buffers: Sequence[Buffer]) -> None:
        self.bind_set_buffers(0, buffers)

    def bind_set_buffers(self, set_index: int, buffers: Sequence[Buffer]) -> None:
        arr = (_vp * len(buffers))(*[b.handle for b in buffers])
        _check(_lib.skyla_hip_pipeline_bind(self._h, set_index, arr, len(buffers)))

    def threads(self) -> tuple[int, int, int]:
        out = (C.c_uint32 * 3)()
        _check(_lib.skyla_hip_pipeline_threads(self._h, out))
        return tuple(out)

    def free(self) -> None:
        if self._h:
            _lib.skyla_hip_pipeline_free(self._h)
            self._h = None


class Recorder:
    """skyla-vk Recorder (record.rs:17-58)."""

    def __init__(self, handle: int):
        self._h = handle

    def dispatch(self, p: Pipeline, groups: Sequence[int], push: Sequence[int]) -> None:
        self.dispatch_set(p, 0, groups, push)

    def dispatch_set(self, p: Pipeline, set_index: int, groups: Sequence[int], push: Sequence[int]) -> None:
        _check(_lib.skyla_hip_record_dispatch(self._h, p._h, set_index, _u32s(groups), _u32s(push), len(push)))

    def barrier(self) -> None:
        _check(_lib.skyla_hip_record_barrier(self._h))

    def host_barrier(self) -> None:
        _check(_lib.skyla_hip_record_host_barrier(self._h))

    def mark(self, label: str) -> None:
        _check(_lib.skyla_hip_record_mark(self._h, label.encode()))


class Recording:
    def __init__(self, ctx: "Context", handle: int):
        self.ctx, self._h = ctx, handle

    def __len__(self) -> int:
        return _lib.skyla_hip_recording_len(self._h)

    def launches(self) -> int:
        """Kernel launches per replay (fused runs of independent dispatches count once)."""
        return _lib.skyla_hip_recording_launches(self._h)

    def free(self) -> None:
        if self._h:
            _lib.skyla_hip_recording_free(self._h)
            self._h = None


class Context:
    """skyla-vk Context (context.rs:85, buffer.rs:59-73, pipeline.rs:6-135, record.rs:82-149)."""

    def __init__(self, device: int = -1):
        load_library()
        h = _vp()
        _check(_lib.skyla_hip_context_new(device, C.byref(h)))
        self._h = h.value
        self.subgroup_size = _lib.skyla_hip_subgroup_size(self._h)

    @classmethod
    def new(cls, device: int = -1) -> "Context":
        return cls(device)

    def max_buffer(self) -> int:
        return _lib.skyla_hip_max_buffer(self._h)

    def device_name(self) -> str:
        buf = C.create_string_buffer(256)
        _check(_lib.skyla_hip_device_name(self._h, buf, 256))
        return buf.value.decode()

    def alloc_host(self, size: int) -> Buffer:
        h = _vp()
        _check(_lib.skyla_hip_alloc(self._h, size, C.byref(h)))
        return Buffer(self, h.value, size)

    def create_pipeline(self, name: str, n_buffers: int, push_size: int, spec: Sequence[int]) -> Pipeline:
        return self.create_pipeline_sets(name, n_buffers, push_size, spec, 1)

    def create_pipeline_sets(self, name: str, n_buffers: int, push_size: int, spec: Sequence[int],
                             n_sets: int) -> Pipeline:
        h = _vp()
        _check(_lib.skyla_hip_pipeline_new(self._h, name.encode(), n_buffers, push_size, _u32s(spec),
                                           len(spec), n_sets, C.byref(h)))
        return Pipeline(self, h.value, name, spec)

    def record(self, profile: bool, f: Callable[[Recorder], None]) -> Recording:
        h = _vp()
        _check(_lib.skyla_hip_record_begin(self._h, int(profile), C.byref(h)))
        r = Recorder(h.value)
        try:
            f(r)
        except BaseException:
            out = _vp()
            _lib.skyla_hip_record_end(h.value, C.byref(out))
            if out.value:
                _lib.skyla_hip_recording_free(out.value)
            raise
        out = _vp()
        _check(_lib.skyla_hip_record_end(h.value, C.byref(out)))
        return Recording(self, out.value)

    def replay(self, rec: Recording) -> None:
        _check(_lib.skyla_hip_replay(self._h, rec._h))

    def replay_timed(self, rec: Recording) -> float:
        ns = C.c_double()
        _check(_lib.skyla_hip_replay_timed(self._h, rec._h, C.byref(ns)))
        return ns.value

    def marks(self, rec: Recording) -> list[tuple[str, float]]:
        count = C.c_uint32()
        _check(_lib.skyla_hip_marks(self._h, rec._h, None, None, 0, C.byref(count)))
        n = count.value
        labels = (C.c_char_p * max(1, n))()
        ns = (C.c_double * max(1, n))()
        _check(_lib.skyla_hip_marks(self._h, rec._h, labels, ns, n, C.byref(count)))
        return [(labels[i].decode(), ns[i]) for i in range(n)]

    def time_dispatch(self, p: Pipeline, groups: Sequence[int], push: Sequence[int], reps: int) -> list[float]:
        out = (C.c_double * reps)()
        _check(_lib.skyla_hip_time_dispatch(self._h, p._h, _u32s(groups), _u32s(push), len(push), reps, out))
        return list(out)

    def dispatch_noalloc(self, p: Pipeline, groups: Sequence[int], push: Sequence[int]) -> None:
        """One synchronous dispatch that allocates no device memory (a K-split matmul takes
        the context's static scratch array; see include/skyla_hip.h)."""
        _check(_lib.skyla_hip_dispatch_noalloc(self._h, p._h, _u32s(groups), _u32s(push), len(push)))

    def free(self) -> None:
        if self._h:
            _lib.skyla_hip_context_free(self._h)
            self._h = None
