"""ctypes binding to ``libktir_hip.so`` (the C ABI in ``include/ktir_hip.h``).

Everything that runs on the GPU goes through this module.  The library is
built in-tree by ``ktir_cpu_amd/build.py``; if it is missing, or no GPU is
visible, :func:`lib` raises, because the backend has no CPU fallback.
Constants (dtype codes, opcodes, predicates) are read from the header itself
so the host and device agree by construction.
"""

from __future__ import annotations

import ctypes as C
import os
import re
import threading
from typing import Dict, List, Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
HEADER = os.path.join(os.path.dirname(_HERE), "include", "ktir_hip.h")
LIB_PATH = os.path.join(_HERE, "libktir_hip.so")


def _read_defines(path: str) -> Dict[str, int]:
    out = {}
    with open(path) as f:
        for line in f:
            m = re.match(r"#define\s+(KTIR_\w+)\s+(-?\d+)", line)
            if m:
                out[m.group(1)] = int(m.group(2))
    return out


K = _read_defines(HEADER)
MAX_DIMS = K["KTIR_MAX_DIMS"]
MAX_LEAVES = K["KTIR_MAX_LEAVES"]
MAX_INSTR = K["KTIR_MAX_INSTR"]
NREG = K["KTIR_NREG"]
MAX_ROW = K["KTIR_MAX_ROW"]

DTYPE_CODE = {"f16": K["KTIR_F16"], "bf16": K["KTIR_BF16"], "f32": K["KTIR_F32"], "i1": K["KTIR_I1"],
              "i32": K["KTIR_I32"], "index": K["KTIR_I32"], "i64": K["KTIR_I64"], "i8": K["KTIR_I8"],
              "i16": K["KTIR_I16"]}
ELEM_BYTES = {"f16": 2, "bf16": 2, "f32": 4, "i1": 1, "i32": 4, "index": 4, "i64": 8, "i8": 1, "i16": 2}
# numpy storage dtype of each KTIR dtype in device memory (bf16 as raw bits)
STORAGE = {"f16": np.float16, "bf16": np.uint16, "f32": np.float32, "i1": np.bool_, "i32": np.int32,
           "index": np.int32, "i64": np.int64, "i8": np.int8, "i16": np.int16}


def op(name: str) -> int:
    return K["KTIR_OP_" + name]


def cmp(name: str) -> int:
    return K["KTIR_CMP_" + name]


class Leaf(C.Structure):
    _fields_ = [("ptr", C.c_uint64), ("base", C.c_int64), ("lane_stride", C.c_int64),
                ("lane_base", C.c_uint64), ("offsets", C.c_uint64), ("offsets_lane_stride", C.c_int64),
                ("strides", C.c_int64 * MAX_DIMS), ("lo", C.c_int64), ("hi", C.c_int64),
                ("winner", C.c_uint64), ("winner_base", C.c_int64), ("dtype", C.c_int32),
                ("flags", C.c_int32)]


class Instr(C.Structure):
    _fields_ = [("op", C.c_int8), ("dst", C.c_int8), ("a", C.c_int8), ("b", C.c_int8), ("c", C.c_int8),
                ("dt", C.c_int8), ("aux", C.c_int16), ("imm", C.c_int32)]


class Prog(C.Structure):
    _fields_ = [("mode", C.c_int32), ("ndim", C.c_int32), ("n_instr", C.c_int32), ("n_leaves", C.c_int32),
                ("n_pf", C.c_int32), ("pf_leaf", C.c_int8 * 4), ("lanes", C.c_int64), ("shape", C.c_int64 * MAX_DIMS), ("lane_scalars", C.c_uint64),
                ("n_lane_scalars", C.c_int64), ("leaves", Leaf * MAX_LEAVES), ("instr", Instr * MAX_INSTR)]


class IAT(C.Structure):
    _fields_ = [("lanes", C.c_int64), ("n", C.c_int64), ("dir", C.c_uint64), ("dir_ls", C.c_int64),
                ("n_ind", C.c_int32), ("pad", C.c_int32), ("idx_ptr", C.c_uint64 * 4),
                ("idx_dtype", C.c_int32 * 4), ("idx_hi", C.c_int64 * 4), ("idx_lo", C.c_int64 * 4),
                ("pos", C.c_uint64 * 4), ("pos_ls", C.c_int64 * 4), ("pos_lane", C.c_uint64 * 4),
                ("stride", C.c_int64 * 4), ("out", C.c_uint64)]


class MM(C.Structure):
    _fields_ = [("lanes", C.c_int64), ("M", C.c_int64), ("N", C.c_int64), ("K", C.c_int64),
                ("ksteps", C.c_int64), ("a", Leaf), ("b", Leaf), ("a_kstep", C.c_int64),
                ("b_kstep", C.c_int64), ("c", Leaf), ("c0", Leaf), ("accumulate", C.c_int32),
                ("round_dt", C.c_int32), ("quads", C.c_uint64), ("n_quads", C.c_int64)]


class RMW(C.Structure):
    _fields_ = [("n_inst", C.c_int64), ("K", C.c_int64), ("D", C.c_int64), ("dst_pos", C.c_uint64),
                ("src_pos", C.c_uint64), ("dst_idx_ptr", C.c_uint64), ("src_idx_ptr", C.c_uint64),
                ("dst_idx_dtype", C.c_int32), ("src_idx_dtype", C.c_int32), ("dst_idx_hi", C.c_int64),
                ("src_idx_hi", C.c_int64), ("dst_ptr", C.c_uint64), ("src_ptr", C.c_uint64),
                ("dst_dtype", C.c_int32), ("src_dtype", C.c_int32), ("dst_base", C.c_int64),
                ("dst_row", C.c_int64), ("dst_col", C.c_int64), ("dst_hi", C.c_int64), ("src_base", C.c_int64),
                ("src_row", C.c_int64), ("src_col", C.c_int64), ("src_hi", C.c_int64), ("op", C.c_int32),
                ("order", C.c_int32), ("dt", C.c_int32), ("pad", C.c_int32), ("n_rows", C.c_int64),
                ("head", C.c_uint64), ("link", C.c_uint64), ("rows", C.c_uint64), ("srcs", C.c_uint64)]


class ATTN(C.Structure):
    _fields_ = [("lanes", C.c_int64), ("M", C.c_int64), ("N", C.c_int64), ("D", C.c_int64),
                ("q_ptr", C.c_uint64), ("k_ptr", C.c_uint64), ("v_ptr", C.c_uint64),
                ("q_base", C.c_uint64), ("k_base", C.c_uint64), ("v_base", C.c_uint64),
                ("q_row", C.c_int64), ("k_row", C.c_int64), ("v_row", C.c_int64),
                ("k_step", C.c_int64), ("v_step", C.c_int64), ("trips", C.c_uint64), ("order", C.c_uint64),
                ("qpos0", C.c_uint64), ("kpos0", C.c_uint64), ("kpos_step", C.c_int64),
                ("scale", C.c_float), ("neg", C.c_float), ("causal", C.c_int32), ("pred", C.c_int32),
                ("dtype", C.c_int32), ("pad", C.c_int32),
                ("m_out", C.c_uint64), ("l_out", C.c_uint64), ("acc_out", C.c_uint64),
                ("o_ptr", C.c_uint64), ("o_base", C.c_uint64), ("o_row", C.c_int64), ("o_dtype", C.c_int32),
                ("v16_ready", C.c_int32), ("v16_ptr", C.c_uint64), ("v16_flag", C.c_uint64), ("v16_lo", C.c_int64),
                ("v16_n", C.c_int64), ("pairs", C.c_uint64), ("n_pairs", C.c_int64)]


class PATTN(C.Structure):
    _fields_ = [("lanes", C.c_int64), ("M", C.c_int64), ("N", C.c_int64), ("D", C.c_int64),
                ("q_ptr", C.c_uint64), ("q_base", C.c_uint64), ("q_row", C.c_int64), ("q_lo", C.c_int64),
                ("q_hi", C.c_int64), ("q_dtype", C.c_int32), ("kv_dtype", C.c_int32),
                ("k_ptr", C.c_uint64), ("v_ptr", C.c_uint64), ("k_base", C.c_uint64), ("v_base", C.c_uint64),
                ("k_row", C.c_int64), ("v_row", C.c_int64), ("k_page", C.c_int64), ("v_page", C.c_int64),
                ("k_lo", C.c_int64), ("k_hi", C.c_int64), ("v_lo", C.c_int64), ("v_hi", C.c_int64),
                ("tbl_ptr", C.c_uint64), ("tbl_pos", C.c_uint64), ("tbl_step", C.c_int64), ("tbl_lo", C.c_int64),
                ("tbl_hi", C.c_int64), ("tbl_dtype", C.c_int32), ("pred", C.c_int32), ("trips", C.c_uint64),
                ("order", C.c_uint64), ("qpos0", C.c_uint64), ("kpos0", C.c_uint64), ("kpos_step", C.c_int64), ("row_div", C.c_int64),
                ("causal", C.c_int32), ("pad", C.c_int32), ("scale", C.c_float), ("neg", C.c_float),
                ("m0", C.c_float), ("l0", C.c_float), ("m_out", C.c_uint64), ("l_out", C.c_uint64),
                ("acc_out", C.c_uint64),
                ("out_ptr", C.c_uint64), ("out_base", C.c_uint64), ("out_grp", C.c_int64),
                ("out_gstride", C.c_int64), ("out_row", C.c_int64), ("out_lo", C.c_int64), ("out_hi", C.c_int64),
                ("out_dtype", C.c_int32), ("out_pad", C.c_int32)]


class KTIRDeviceError(RuntimeError):
    pass


_lib = None
_lock = threading.Lock()


def lib():
    """Load the HIP library and initialise device 0 (raises when unavailable)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m ktir_cpu_amd.build` "
                               "(the KTIR GPU backend has no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        L.ktir_last_error.restype = C.c_char_p
        for name in ("ktir_init", "ktir_malloc", "ktir_free", "ktir_memcpy_h2d", "ktir_memcpy_d2h",
                     "ktir_memcpy_d2d", "ktir_memset", "ktir_sync", "ktir_check_error_flag",
                     "ktir_launch_program", "ktir_scatter_winners", "ktir_iat_offsets",
                     "ktir_launch_matmul", "ktir_event_create", "ktir_event_record",
                     "ktir_event_elapsed_ms", "ktir_event_destroy", "ktir_device_info",
                     "ktir_launch_row_rmw", "ktir_launch_attention", "ktir_rmw_variant", "ktir_shutdown", "ktir_set_row_grid_limit",
                     "ktir_launch_row_rmw_noalloc", "ktir_launch_paged_attention"):
            getattr(L, name).restype = C.c_int
        L.ktir_malloc.argtypes = [C.c_uint64, C.POINTER(C.c_uint64)]
        L.ktir_free.argtypes = [C.c_uint64]
        L.ktir_memcpy_h2d.argtypes = [C.c_uint64, C.c_void_p, C.c_uint64]
        L.ktir_memcpy_d2h.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64]
        L.ktir_memcpy_d2d.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        L.ktir_memset.argtypes = [C.c_uint64, C.c_int, C.c_uint64]
        L.ktir_launch_program.argtypes = [C.POINTER(Prog)]
        L.ktir_scatter_winners.argtypes = [C.POINTER(Leaf), C.c_int64, C.c_int64, C.c_uint64]
        L.ktir_iat_offsets.argtypes = [C.POINTER(IAT)]
        L.ktir_launch_matmul.argtypes = [C.POINTER(MM)]
        L.ktir_launch_row_rmw.argtypes = [C.POINTER(RMW)]
        L.ktir_rmw_variant.argtypes = [C.POINTER(RMW)]
        L.ktir_launch_row_rmw_noalloc.argtypes = [C.POINTER(RMW)]
        L.ktir_set_row_grid_limit.argtypes = [C.c_int64]
        L.ktir_launch_attention.argtypes = [C.POINTER(ATTN)]
        L.ktir_launch_paged_attention.argtypes = [C.POINTER(PATTN)]
        L.ktir_event_create.argtypes = [C.POINTER(C.c_uint64)]
        L.ktir_event_record.argtypes = [C.c_uint64]
        L.ktir_event_elapsed_ms.argtypes = [C.c_uint64, C.c_uint64, C.POINTER(C.c_float)]
        L.ktir_event_destroy.argtypes = [C.c_uint64]
        L.ktir_device_info.argtypes = [C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int64),
                                       C.c_char_p, C.c_int]
        rc = L.ktir_init(int(os.environ.get("KTIR_DEVICE", "0")))
        if rc != 0:
            raise RuntimeError("KTIR GPU backend: no usable HIP device: "
                               + L.ktir_last_error().decode(errors="replace"))
        _lib = L
        return _lib


def check(rc: int, what: str = ""):
    if rc == 0:
        return
    msg = lib().ktir_last_error().decode(errors="replace")
    if what:
        msg = f"{what}: {msg}"
    if rc == K["KTIR_E_INDEX"]:
        raise IndexError(msg)
    if rc == K["KTIR_E_ARG"]:
        raise ValueError(msg)
    if rc == K["KTIR_E_UNSUPPORTED"]:
        raise NotImplementedError(msg)
    raise KTIRDeviceError(msg)


def set_row_grid_limit(max_workgroups: int):
    """Bound the workgroups of row-program launches (0: no bound)."""
    check(lib().ktir_set_row_grid_limit(int(max_workgroups)), "ktir_set_row_grid_limit")


def device_info() -> dict:
    cu, clk, mem = C.c_int(), C.c_int(), C.c_int64()
    name = C.create_string_buffer(256)
    check(lib().ktir_device_info(C.byref(cu), C.byref(clk), C.byref(mem), name, 256))
    return {"cu_count": cu.value, "clock_khz": clk.value, "hbm_bytes": mem.value,
            "name": name.value.decode(errors="replace")}


class DeviceBuffer:
    """One device allocation; freed explicitly or when garbage collected."""

    __slots__ = ("ptr", "nbytes", "_pool", "host_writes", "__weakref__")

    def __init__(self, nbytes: int, pool: Optional["BufferPool"] = None):
        p = C.c_uint64()
        check(lib().ktir_malloc(max(int(nbytes), 1), C.byref(p)), "ktir_malloc")
        self.ptr = p.value
        self.nbytes = int(nbytes)
        self._pool = pool
        self.host_writes = 0         # uploads and fills from the host so far (device copies it caches check it)

    def free(self):
        if self.ptr:
            check(lib().ktir_free(self.ptr), "ktir_free")
            self.ptr = 0

    def upload(self, arr: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(arr)
        assert offset + a.nbytes <= self.nbytes
        self.host_writes += 1
        check(lib().ktir_memcpy_h2d(self.ptr + offset, a.ctypes.data, a.nbytes), "ktir_memcpy_h2d")

    def download_into(self, dst: np.ndarray, offset: int = 0):
        """Copy dst.nbytes bytes from the buffer (at `offset`) into the
        C-contiguous host array `dst`."""
        assert dst.flags.c_contiguous and offset + dst.nbytes <= self.nbytes
        check(lib().ktir_memcpy_d2h(dst.ctypes.data, self.ptr + offset, dst.nbytes), "ktir_memcpy_d2h")

    def memset(self, value: int = 0, offset: int = 0, nbytes: Optional[int] = None):
        n = self.nbytes - offset if nbytes is None else int(nbytes)
        assert offset + n <= self.nbytes
        self.host_writes += 1
        check(lib().ktir_memset(self.ptr + offset, int(value), n), "ktir_memset")

    def download(self, nbytes: int, offset: int = 0) -> bytes:
        out = np.empty(nbytes, dtype=np.uint8)
        check(lib().ktir_memcpy_d2h(out.ctypes.data, self.ptr + offset, nbytes), "ktir_memcpy_d2h")
        return out


class BufferPool:
    """Size-bucketed reuse of device buffers (all work is on one stream, so a
    buffer released by the host can be handed to a later launch)."""

    def __init__(self):
        self._free: Dict[int, List[DeviceBuffer]] = {}
        self.live: List[DeviceBuffer] = []
        self.bytes_allocated = 0

    @staticmethod
    def _bucket(n: int) -> int:
        n = max(int(n), 256)
        return 1 << (n - 1).bit_length() if n < (1 << 20) else ((n + (1 << 20) - 1) >> 20) << 20

    def get(self, nbytes: int) -> DeviceBuffer:
        b = self._bucket(nbytes)
        lst = self._free.get(b)
        if lst:
            return lst.pop()
        buf = DeviceBuffer(b)
        self.bytes_allocated += b
        self.live.append(buf)
        return buf

    def put(self, buf: DeviceBuffer):
        self._free.setdefault(buf.nbytes, []).append(buf)

    def release_all(self):
        for b in self.live:
            b.free()
        self.live.clear()
        self._free.clear()
        self.bytes_allocated = 0


def sync():
    check(lib().ktir_sync(), "ktir_sync")
    check(lib().ktir_check_error_flag(), "device")


class Event:
    def __init__(self):
        e = C.c_uint64()
        check(lib().ktir_event_create(C.byref(e)))
        self.ev = e.value

    def record(self):
        check(lib().ktir_event_record(self.ev))

    def elapsed_ms(self, later: "Event") -> float:
        ms = C.c_float()
        check(lib().ktir_event_elapsed_ms(self.ev, later.ev, C.byref(ms)))
        return float(ms.value)

    def __del__(self):
        try:
            if _lib is not None and self.ev:
                _lib.ktir_event_destroy(self.ev)
        except Exception:
            pass
