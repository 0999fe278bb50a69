"""ctypes binding of libspkv2_mi355x.so.

`Model` mirrors the reference's ctypes driver
(research/reliability/runtime_driver.py:44-128): load -> prepare -> set input
-> run -> get output, same return-code checks.  Loading fails loudly when the
library has not been built: there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libspkv2_mi355x.so"


class FaultEvent(ctypes.Structure):
    _fields_ = [("node_id", ctypes.c_uint32), ("tensor_id", ctypes.c_uint32), ("element_index", ctypes.c_uint64),
                ("bit_index", ctypes.c_uint8), ("invocation_index", ctypes.c_uint32), ("seed", ctypes.c_uint64),
                ("enabled", ctypes.c_int)]


class ReliabilityStats(ctypes.Structure):
    _fields_ = [("injected_faults", ctypes.c_uint64), ("detected_faults", ctypes.c_uint64),
                ("recovered_faults", ctypes.c_uint64), ("unrecovered_faults", ctypes.c_uint64),
                ("rerun_count", ctypes.c_uint64)]


class RangeObservation(ctypes.Structure):
    _fields_ = [("node_id", ctypes.c_uint32), ("tensor_id", ctypes.c_uint32), ("observed_min", ctypes.c_float),
                ("observed_max", ctypes.c_float), ("observations", ctypes.c_uint64)]


# name -> (restype, argtypes) for every entry point of include/*.h
VP, I, U32, SZ, CP = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_size_t, ctypes.c_char_p
SIGNATURES = {
    # spkv2_runtime.h
    "spkv2_runtime_version": (CP, []),
    "spkv2_load_file": (I, [CP, ctypes.POINTER(VP)]),
    "spkv2_load_memory": (I, [VP, SZ, ctypes.POINTER(VP)]),
    "spkv2_prepare": (I, [VP, VP, SZ]),
    "spkv2_prepare_with_scratch": (I, [VP, VP, SZ, VP, SZ]),
    "spkv2_set_input": (I, [VP, I, VP, SZ]),
    "spkv2_bind_input": (I, [VP, I, VP, SZ]),
    "spkv2_bind_output": (I, [VP, I, VP, SZ]),
    "spkv2_get_output_size": (I, [VP, I, ctypes.POINTER(SZ)]),
    "spkv2_get_output": (I, [VP, I, VP, SZ]),
    "spkv2_run": (I, [VP]),
    "spkv2_set_fault_event": (I, [VP, ctypes.POINTER(FaultEvent)]),
    "spkv2_clear_fault_event": (None, [VP]),
    "spkv2_get_reliability_stats": (I, [VP, ctypes.POINTER(ReliabilityStats)]),
    "spkv2_reset_reliability_stats": (None, [VP]),
    "spkv2_get_range_observation": (I, [VP, U32, ctypes.POINTER(RangeObservation)]),
    "spkv2_reset_range_observations": (None, [VP]),
    "spkv2_profile_dump": (None, []),
    "spkv2_free": (None, [VP]),
    "spkv2_register_kernel": (I, [ctypes.c_uint16, ctypes.c_uint16, ctypes.c_uint16, VP, I]),
    "spkv2_clear_user_kernels": (None, []),
    # spkv2_platform.h
    "spkv2_platform_malloc": (VP, [SZ]),
    "spkv2_platform_calloc": (VP, [SZ, SZ]),
    "spkv2_platform_free": (None, [VP]),
    "spkv2_set_num_threads": (None, [I]),
    "spkv2_get_num_threads": (I, []),
    "spkv2_set_gemm_tiling": (None, [I, I]),
    "spkv2_get_gemm_kc": (I, []),
    "spkv2_get_gemm_nc": (I, []),
    "spkv2_auto_tune_gemm": (None, [I, I]),
    "spkv2_set_parallel_cost_threshold": (None, [I]),
    "spkv2_get_parallel_cost_threshold": (I, []),
    "spkv2_should_parallelize": (I, [I, I]),
    "spkv2_detect_topology": (None, []),
    "spkv2_get_topology": (VP, []),
    "spkv2_set_affinity": (None, [I]),
    # spkv2_mi355x.h
    "spkv2_mi355x_fp16_to_fp32": (None, [VP, VP, SZ]),
    "spkv2_ctx_tensor_record": (VP, [VP, U32]),
    "spkv2_ctx_tensor_data": (VP, [VP, U32]),
    "spkv2_ctx_get_attr": (I, [VP, VP, VP]),
    "spkv2_ctx_stream": (VP, [VP]),
    "spkv2_ctx_find_quant_param": (VP, [VP, U32]),
    "spkv2_ctx_quant_scales": (VP, [VP, VP]),
    "spkv2_ctx_quant_zero_points": (VP, [VP, VP]),
    "spkv2_ctx_node_cache": (I, [VP, U32, VP, VP]),
    "spkv2_device_malloc": (I, [ctypes.POINTER(VP), SZ]),
    "spkv2_device_free": (I, [VP]),
    "spkv2_device_memcpy_h2d": (I, [VP, VP, SZ]),
    "spkv2_device_memcpy_d2h": (I, [VP, VP, SZ]),
    "spkv2_device_memcpy_d2d": (I, [VP, VP, SZ]),
    "spkv2_device_synchronize": (I, []),
    "spkv2_device_info": (I, [ctypes.POINTER(I), ctypes.c_char_p, SZ]),
    "spkv2_mi355x_last_error": (CP, []),
    "spkv2_fnv1a32": (U32, [ctypes.c_char_p, SZ]),
    "spkv2_mi355x_set_graph_mode": (I, [VP, I]),
    "spkv2_mi355x_set_profiling": (I, [VP, I]),
    "spkv2_mi355x_node_time": (I, [VP, U32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(U32)]),
    "spkv2_mi355x_reset_node_times": (None, [VP]),
    "spkv2_mi355x_node_kernel_name": (I, [VP, U32, ctypes.c_char_p, SZ]),
    "spkv2_mi355x_conv_int8_accumulators": (I, [VP, U32, VP, SZ]),
    "spkv2_mi355x_set_int8_capture": (I, [VP, I]),
    "spkv2_mi355x_conv_int8_accumulators_noalloc": (I, [VP, U32, VP, SZ]),
    "spkv2_mi355x_read_int8_tensor": (I, [VP, U32, VP, SZ]),
}

_LIB = None


def load_library(path: str | Path | None = None) -> ctypes.CDLL:
    """Loads and types the MI355X runtime.  Raises if it is not built."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is not built; run `python -m spinnv2_amd.build` (no CPU fallback exists)")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


class RuntimeError_(RuntimeError):
    def __init__(self, action: str, code: int, detail: str = "") -> None:
        super().__init__(f"SPINNV2 mi355x runtime {action} failed with {code}" + (f": {detail}" if detail else ""))
        self.code = code


def _check(lib, code: int, action: str) -> None:
    if code != 0:
        raise RuntimeError_(action, code, lib.spkv2_mi355x_last_error().decode(errors="replace"))


class DeviceBuffer:
    """A hipMalloc'd buffer owned from Python (for bind_input / bind_output)."""

    def __init__(self, nbytes: int, lib=None) -> None:
        self.lib = lib or load_library()
        self.nbytes = int(nbytes)
        self.ptr = ctypes.c_void_p()
        _check(self.lib, self.lib.spkv2_device_malloc(ctypes.byref(self.ptr), self.nbytes), "device malloc")

    def upload(self, array: np.ndarray) -> None:
        a = np.ascontiguousarray(array)
        assert a.nbytes == self.nbytes
        _check(self.lib, self.lib.spkv2_device_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes), "h2d")

    def download(self, dtype=np.float32) -> np.ndarray:
        out = np.empty(self.nbytes // np.dtype(dtype).itemsize, dtype=dtype)
        _check(self.lib, self.lib.spkv2_device_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes), "d2h")
        return out

    def free(self) -> None:
        if self.ptr:
            self.lib.spkv2_device_free(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self) -> None:  # pragma: no cover - best effort
        try:
            self.free()
        except Exception:
            pass


class Model:
    """One SPK package loaded and prepared on the current GPU."""

    def __init__(self, spk: bytes | str | Path, *, prepare: bool = True, lib=None) -> None:
        self.lib = lib or load_library()
        self.ctx = ctypes.c_void_p()
        if isinstance(spk, (bytes, bytearray)):
            self._blob = ctypes.create_string_buffer(bytes(spk), len(spk))  # must outlive the context
            _check(self.lib, self.lib.spkv2_load_memory(self._blob, len(spk), ctypes.byref(self.ctx)), "load")
        else:
            self._blob = None
            _check(self.lib, self.lib.spkv2_load_file(str(spk).encode(), ctypes.byref(self.ctx)), "load")
        if prepare:
            self.prepare()

    def prepare(self) -> None:
        _check(self.lib, self.lib.spkv2_prepare(self.ctx, None, 0), "prepare")

    def prepare_with_scratch(self, arena: DeviceBuffer | None = None, scratch: DeviceBuffer | None = None) -> int:
        """spkv2_prepare_with_scratch with caller-owned device buffers (None:
        the runtime allocates that one).  Returns the entry point's code."""
        return self.lib.spkv2_prepare_with_scratch(self.ctx, arena.ptr if arena else None, arena.nbytes if arena else 0,
                                                   scratch.ptr if scratch else None, scratch.nbytes if scratch else 0)

    def set_input(self, index: int, array: np.ndarray) -> None:
        a = np.ascontiguousarray(array, dtype=np.float32)
        _check(self.lib, self.lib.spkv2_set_input(self.ctx, index, a.ctypes.data, a.nbytes), "set input")

    def bind_input(self, index: int, buf: DeviceBuffer) -> None:
        _check(self.lib, self.lib.spkv2_bind_input(self.ctx, index, buf.ptr, buf.nbytes), "bind input")

    def bind_output(self, index: int, buf: DeviceBuffer) -> None:
        _check(self.lib, self.lib.spkv2_bind_output(self.ctx, index, buf.ptr, buf.nbytes), "bind output")

    def run(self) -> None:
        _check(self.lib, self.lib.spkv2_run(self.ctx), "run")

    def run_rc(self) -> int:
        """spkv2_run's return code as is (fault-event errors are negative)."""
        return self.lib.spkv2_run(self.ctx)

    def output_size(self, index: int = 0) -> int:
        size = ctypes.c_size_t()
        _check(self.lib, self.lib.spkv2_get_output_size(self.ctx, index, ctypes.byref(size)), "output size")
        return size.value

    def get_output(self, index: int = 0) -> np.ndarray:
        out = np.empty(self.output_size(index) // 4, dtype=np.float32)
        _check(self.lib, self.lib.spkv2_get_output(self.ctx, index, out.ctypes.data, out.nbytes), "get output")
        return out

    def __call__(self, *inputs: np.ndarray) -> np.ndarray:
        for i, a in enumerate(inputs):
            self.set_input(i, a)
        self.run()
        return self.get_output(0)

    def set_graph_mode(self, on: bool) -> None:
        _check(self.lib, self.lib.spkv2_mi355x_set_graph_mode(self.ctx, int(on)), "graph mode")

    def set_profiling(self, on: bool) -> None:
        _check(self.lib, self.lib.spkv2_mi355x_set_profiling(self.ctx, int(on)), "profiling")

    def node_time(self, node_id: int) -> tuple[float, int]:
        ms, cnt = ctypes.c_double(), ctypes.c_uint32()
        _check(self.lib, self.lib.spkv2_mi355x_node_time(self.ctx, node_id, ctypes.byref(ms), ctypes.byref(cnt)),
               "node time")
        return ms.value, cnt.value

    def reset_node_times(self) -> None:
        self.lib.spkv2_mi355x_reset_node_times(self.ctx)

    def kernel_name(self, node_id: int) -> str:
        buf = ctypes.create_string_buffer(128)
        _check(self.lib, self.lib.spkv2_mi355x_node_kernel_name(self.ctx, node_id, buf, 128), "kernel name")
        return buf.value.decode()

    def set_int8_capture(self, on: bool) -> None:
        """Every later run also keeps each INT8 conv's raw int32 accumulators
        (read back with int8_accumulators)."""
        _check(self.lib, self.lib.spkv2_mi355x_set_int8_capture(self.ctx, 1 if on else 0), "int8 capture")

    def int8_accumulators(self, node_id: int, nbytes: int) -> np.ndarray:
        out = np.empty(nbytes // 4, dtype=np.int32)
        _check(self.lib, self.lib.spkv2_mi355x_conv_int8_accumulators(self.ctx, node_id, out.ctypes.data, nbytes),
               "int8 accumulators")
        return out

    def read_int8_tensor(self, tensor_id: int, shape) -> np.ndarray:
        """An int8 activation tensor (the INT8 configuration with int8
        tensors between nodes) after a run, as an NCHW int8 array."""
        out = np.empty(tuple(int(d) for d in shape), dtype=np.int8)
        _check(self.lib, self.lib.spkv2_mi355x_read_int8_tensor(self.ctx, tensor_id, out.ctypes.data, out.nbytes),
               "read int8 tensor")
        return out

    def set_fault_event(self, event: FaultEvent | dict | None) -> int:
        """Arms one bit flip (a FaultEvent or a dict of its fields); None
        clears it.  Returns the entry point's code."""
        if event is None:
            self.lib.spkv2_clear_fault_event(self.ctx)
            return 0
        if isinstance(event, dict):
            event = FaultEvent(**event)
        return self.lib.spkv2_set_fault_event(self.ctx, ctypes.byref(event))

    def reliability_stats(self) -> dict:
        s = ReliabilityStats()
        _check(self.lib, self.lib.spkv2_get_reliability_stats(self.ctx, ctypes.byref(s)), "stats")
        return {name: int(getattr(s, name)) for name, _ in s._fields_}

    def reset_reliability_stats(self) -> None:
        self.lib.spkv2_reset_reliability_stats(self.ctx)

    def range_observation(self, node_id: int) -> dict:
        o = RangeObservation()
        _check(self.lib, self.lib.spkv2_get_range_observation(self.ctx, node_id, ctypes.byref(o)), "range observation")
        return {name: getattr(o, name) for name, _ in o._fields_}

    def reset_range_observations(self) -> None:
        self.lib.spkv2_reset_range_observations(self.ctx)

    def close(self) -> None:
        if self.ctx:
            self.lib.spkv2_free(self.ctx)
            self.ctx = ctypes.c_void_p()

    def __enter__(self) -> "Model":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass


def device_available() -> bool:
    lib = load_library()
    cus = ctypes.c_int()
    return lib.spkv2_device_info(ctypes.byref(cus), None, 0) == 0 and cus.value > 0
