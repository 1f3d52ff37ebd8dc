"""The reference's simulated HBM surface over the device arena.

Callers of the reference seed memory at literal stick addresses and read it
back after a run through ``interp.memory.hbm`` (``HBMSimulator``,
reference ``memory.py:311-398``), after replacing
``KTIRInterpreter._prepare_execution(grid)`` with a version that calls the
original and then writes (``tests/test_indirect_access.py:30-46``,
``tests/test_examples.py:664-674``).  ``DeviceHBM`` keeps that surface:

* before a run, ``write`` stages host data at a byte address (a new
  allocation there, or into the staged allocation that holds the address),
  and ``allocate`` hands out stick-aligned addresses from 0x10000 as the
  reference's allocator does, which is where ``execute_function`` places its
  array arguments;
* the run places every staged allocation in the device arena at its address;
* after the run, ``read`` and ``write`` go to the device arena.

Reads are value reads relative to the allocation that holds the start
address, zero past its end; a start address in no allocation raises
``ValueError`` (reference ``memory.py:190-266``).
"""

from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import numpy as np

from . import runtime as rt
from .executor import HBM_BASE, STICK_BYTES


class DeviceHBM:
    STICK_BYTES = STICK_BYTES

    def __init__(self, size_gb: int = 128):
        self.size_gb = size_gb
        self.size_bytes = size_gb * 1024 * 1024 * 1024
        self.next_ptr = HBM_BASE
        self._staged: Dict[int, np.ndarray] = {}
        self._arena = None
        self._np_dtypes: Dict[str, np.dtype] = {}

    # -- allocation ----------------------------------------------------------
    def allocate(self, size: int) -> int:
        """Stick index of `size` fresh bytes (reference memory.py:336-352)."""
        ptr = self.next_ptr
        self.next_ptr = (ptr + int(size) + STICK_BYTES - 1) & ~(STICK_BYTES - 1)
        return ptr // STICK_BYTES

    def staged(self) -> List[Tuple[int, np.ndarray]]:
        return sorted(self._staged.items())

    def attach(self, arena, np_dtypes: Dict[str, np.dtype]):
        """The run placed memory on the device: reads and writes go there.
        `np_dtypes`: the host dtype of each allocation, by name."""
        self._arena = arena
        self._np_dtypes = np_dtypes

    # -- lookup ----------------------------------------------------------------
    def _find_staged(self, ptr: int) -> Optional[Tuple[int, np.ndarray]]:
        if ptr in self._staged:
            return ptr, self._staged[ptr]
        for base, arr in self._staged.items():
            if base < ptr < base + arr.nbytes:
                return base, arr
        return None

    def _device_alloc(self, ptr: int):
        try:
            a = self._arena.find(ptr)
        except ValueError:
            return None
        return a

    def _device_array(self, a) -> np.ndarray:
        rt.sync()
        raw = self._arena.buf.download(a.nbytes, a.off)
        return np.frombuffer(raw.tobytes(), dtype=self._np_dtypes.get(a.name, rt.STORAGE[a.dtype])).copy()

    # -- reference surface -------------------------------------------------------
    def read(self, stick: int, n_elements: int, dtype: str, *, intra_byte: int = 0,
             offsets: Optional[np.ndarray] = None) -> np.ndarray:
        assert 0 <= intra_byte < STICK_BYTES
        ptr = int(stick) * STICK_BYTES + intra_byte
        npd = rt.STORAGE[dtype]
        esz = rt.ELEM_BYTES[dtype]   # the element offset counts the requested dtype (reference memory.py:210)
        if self._arena is not None:
            a = self._device_alloc(ptr)
            if a is None:
                raise ValueError(f"Read from unmapped address 0x{ptr:x} (n_elements={n_elements})")
            flat, base = self._device_array(a), a.addr
        else:
            hit = self._find_staged(ptr)
            if hit is None:
                raise ValueError(f"Read from unmapped address 0x{ptr:x} (n_elements={n_elements})")
            base, flat = hit[0], hit[1].reshape(-1)
        off = (ptr - base) // esz
        if offsets is not None:
            idx = off + np.asarray(offsets, dtype=np.int64)
            oob = idx >= flat.size
            out = flat[np.where(oob, 0, idx)].copy()
            out[oob] = 0
            return out
        out = np.zeros(int(n_elements), dtype=npd)
        avail = max(0, min(int(n_elements), flat.size - off))
        out[:avail] = flat[off:off + avail].astype(npd)
        return out

    def write(self, stick: int, data: np.ndarray, *, intra_byte: int = 0, offsets: Optional[np.ndarray] = None):
        assert 0 <= intra_byte < STICK_BYTES
        ptr = int(stick) * STICK_BYTES + intra_byte
        src = np.asarray(data).reshape(-1)
        if self._arena is not None:
            a = self._device_alloc(ptr)
            if a is None:
                raise NotImplementedError(f"HBM write to 0x{ptr:x} after the run, outside every allocation")
            flat = self._device_array(a)
            self._put(flat, (ptr - a.addr) // src.itemsize, src, offsets)
            self._arena.buf.upload(flat.view(np.uint8), a.off)
            return
        hit = self._find_staged(ptr)
        if hit is None:
            if offsets is not None:
                raise ValueError(f"Scatter to unmapped address 0x{ptr:x}")
            self._staged[ptr] = src.copy()
            return
        base, arr = hit
        self._put(arr, (ptr - base) // src.itemsize, src, offsets)

    @staticmethod
    def _put(flat: np.ndarray, off: int, src: np.ndarray, offsets):
        if offsets is not None:
            idx = off + np.asarray(offsets, dtype=np.int64)
            keep = idx < flat.size
            flat[idx[keep]] = src[keep]
            return
        fit = max(0, min(src.size, flat.size - off))
        flat[off:off + fit] = src[:fit]


class DeviceMemory:
    """``interp.memory`` (the reference's SpyreMemoryHierarchy,
    ``memory.py:449-463``): the HBM surface; per-core LX lives on the device
    inside the kernels and is accounted by the executor."""

    def __init__(self, num_cores: int, lx_size_mb: int = 2):
        self.num_cores = num_cores
        self.lx_size_mb = lx_size_mb
        self.hbm = DeviceHBM()
