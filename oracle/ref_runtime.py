"""ctypes driver for the reference SPINNV2 C runtime built from its own
sources into oracle/_ref/libspkv2_ref.so (see oracle/Makefile).

TEST INFRASTRUCTURE ONLY: used by tests/ (golden vectors, checking the
oracle restatement), by __graft_entry__.smoke() and by bench.py's CPU
baseline leg.  The product never loads it.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

REF_LIB = Path(__file__).resolve().parent / "_ref" / "libspkv2_ref.so"


# runtime/include/spkv2_runtime.h:13-38
class RefFaultEvent(ctypes.Structure):
    _fields_ = [("node_id", ctypes.c_uint32), ("tensor_id", ctypes.c_uint32), ("element_index", ctypes.c_uint64),
                ("bit_index", ctypes.c_uint8), ("invocation_index", ctypes.c_uint32), ("seed", ctypes.c_uint64),
                ("enabled", ctypes.c_int)]


class RefReliabilityStats(ctypes.Structure):
    _fields_ = [("injected_faults", ctypes.c_uint64), ("detected_faults", ctypes.c_uint64),
                ("recovered_faults", ctypes.c_uint64), ("unrecovered_faults", ctypes.c_uint64),
                ("rerun_count", ctypes.c_uint64)]


class RefRangeObservation(ctypes.Structure):
    _fields_ = [("node_id", ctypes.c_uint32), ("tensor_id", ctypes.c_uint32), ("observed_min", ctypes.c_float),
                ("observed_max", ctypes.c_float), ("observations", ctypes.c_uint64)]


def available() -> bool:
    return REF_LIB.exists()


class RefModel:
    """load_memory -> prepare -> set_input -> run -> get_output on the CPU."""

    def __init__(self, spk: bytes) -> None:
        if not REF_LIB.exists():
            raise FileNotFoundError(f"{REF_LIB} not built (make -C oracle ref)")
        lib = ctypes.CDLL(str(REF_LIB))
        vp = ctypes.c_void_p
        lib.spkv2_load_memory.argtypes = [vp, ctypes.c_size_t, ctypes.POINTER(vp)]
        lib.spkv2_prepare.argtypes = [vp, vp, ctypes.c_size_t]
        lib.spkv2_set_input.argtypes = [vp, ctypes.c_int, vp, ctypes.c_size_t]
        lib.spkv2_run.argtypes = [vp]
        lib.spkv2_get_output_size.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t)]
        lib.spkv2_get_output.argtypes = [vp, ctypes.c_int, vp, ctypes.c_size_t]
        lib.spkv2_free.argtypes = [vp]
        lib.spkv2_set_fault_event.argtypes = [vp, ctypes.POINTER(RefFaultEvent)]
        lib.spkv2_clear_fault_event.argtypes = [vp]
        lib.spkv2_clear_fault_event.restype = None
        lib.spkv2_get_reliability_stats.argtypes = [vp, ctypes.POINTER(RefReliabilityStats)]
        lib.spkv2_get_range_observation.argtypes = [vp, ctypes.c_uint32, ctypes.POINTER(RefRangeObservation)]
        self.lib = lib
        self._blob = ctypes.create_string_buffer(bytes(spk), len(spk))
        self.ctx = vp()
        rc = lib.spkv2_load_memory(self._blob, len(spk), ctypes.byref(self.ctx))
        if rc != 0:
            raise RuntimeError(f"reference load failed: {rc}")
        rc = lib.spkv2_prepare(self.ctx, None, 0)
        if rc != 0:
            raise RuntimeError(f"reference prepare failed: {rc}")

    def run(self, *inputs: np.ndarray, output: int = 0) -> np.ndarray:
        for i, a in enumerate(inputs):
            a = np.ascontiguousarray(a, dtype=np.float32)
            rc = self.lib.spkv2_set_input(self.ctx, i, a.ctypes.data, a.nbytes)
            if rc != 0:
                raise RuntimeError(f"reference set_input failed: {rc}")
        rc = self.lib.spkv2_run(self.ctx)
        if rc != 0:
            raise RuntimeError(f"reference run failed: {rc}")
        size = ctypes.c_size_t()
        self.lib.spkv2_get_output_size(self.ctx, output, ctypes.byref(size))
        out = np.empty(size.value // 4, dtype=np.float32)
        rc = self.lib.spkv2_get_output(self.ctx, output, out.ctypes.data, out.nbytes)
        if rc != 0:
            raise RuntimeError(f"reference get_output failed: {rc}")
        return out

    def set_input(self, index: int, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a, dtype=np.float32)
        return self.lib.spkv2_set_input(self.ctx, index, a.ctypes.data, a.nbytes)

    def run_rc(self) -> int:
        return self.lib.spkv2_run(self.ctx)

    def output(self, index: int = 0) -> np.ndarray:
        size = ctypes.c_size_t()
        self.lib.spkv2_get_output_size(self.ctx, index, ctypes.byref(size))
        out = np.empty(size.value // 4, dtype=np.float32)
        rc = self.lib.spkv2_get_output(self.ctx, index, out.ctypes.data, out.nbytes)
        if rc != 0:
            raise RuntimeError(f"reference get_output failed: {rc}")
        return out

    def set_fault_event(self, event: dict | None) -> int:
        """`event` holds the Spkv2FaultEvent fields; None clears it."""
        if event is None:
            self.lib.spkv2_clear_fault_event(self.ctx)
            return 0
        ev = RefFaultEvent(**event)
        return self.lib.spkv2_set_fault_event(self.ctx, ctypes.byref(ev))

    def reliability_stats(self) -> dict:
        s = RefReliabilityStats()
        rc = self.lib.spkv2_get_reliability_stats(self.ctx, ctypes.byref(s))
        if rc != 0:
            raise RuntimeError(f"reference stats failed: {rc}")
        return {name: int(getattr(s, name)) for name, _ in s._fields_}

    def range_observation(self, node_id: int) -> dict:
        o = RefRangeObservation()
        rc = self.lib.spkv2_get_range_observation(self.ctx, node_id, ctypes.byref(o))
        if rc != 0:
            raise RuntimeError(f"reference range observation failed: {rc}")
        return {name: getattr(o, name) for name, _ in o._fields_}

    def close(self) -> None:
        if self.ctx:
            self.lib.spkv2_free(self.ctx)
            self.ctx = ctypes.c_void_p()

    def __del__(self) -> None:  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass
