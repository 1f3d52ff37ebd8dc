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


class DeviceLX:
    """``interp.memory.get_lx(core)`` (the reference's LXScratchpad,
    ``memory.py:400-446``): byte addresses from 0 in the core's scratchpad.

    Before a run, ``write`` stages data as the reference's allocation store
    does (a new allocation at an unmapped address, else into the allocation
    that holds it, truncated at its end) and ``read`` reads it back.  The run
    places the staged bytes in the core's part of the device LX space; after
    it, ``read`` and ``write`` address that part directly: the scratchpad is
    a flat byte array there, bytes never written read zero, and an address
    past its capacity raises ``ValueError``."""

    def __init__(self, core_id: int, size_mb: int = 2):
        self.core_id = core_id
        self.size_mb = size_mb
        self.capacity = size_mb * 1024 * 1024
        self.used = 0
        self.next_ptr = 0
        self._staged: Dict[int, np.ndarray] = {}
        self._space = None

    def staged(self) -> List[Tuple[int, np.ndarray]]:
        return sorted(self._staged.items())

    def attach(self, space):
        """`space`: the run's LX space (executor.LXSpace), or None."""
        self._space = space

    def _find_staged(self, ptr: int):
        if ptr in self._staged:
            return ptr, self._staged[ptr]
        for base, arr in self._staged.items():
            if base < ptr < base + arr.nbytes:
                return base, arr
        return None

    def _device_bytes(self, ptr: int, nbytes: int) -> np.ndarray:
        sp = self._space
        if ptr < 0 or ptr + nbytes > sp.bytes_per_core:
            raise ValueError(f"LX address 0x{ptr:x}+{nbytes} outside the {sp.bytes_per_core}-byte scratchpad")
        rt.sync()
        return np.asarray(sp.buf.download(nbytes, self.core_id * sp.bytes_per_core + ptr))

    def read(self, ptr: int, n_elements: int, dtype: str, *, offsets: Optional[np.ndarray] = None) -> np.ndarray:
        npd = rt.STORAGE[dtype]
        esz = rt.ELEM_BYTES[dtype]
        if self._space is not None:
            if offsets is not None:
                idx = np.asarray(offsets, dtype=np.int64)
                n = int(idx.max()) + 1 if idx.size else 0
                flat = self._device_bytes(ptr, n * esz).view(npd)
                return flat[idx].copy()
            return self._device_bytes(ptr, int(n_elements) * esz).view(npd).copy()
        hit = self._find_staged(ptr)
        if hit is None:
            raise ValueError(f"Read from unmapped address 0x{ptr:x} (n_elements={n_elements})")
        base, arr = hit
        flat = arr.reshape(-1)
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

    def write(self, ptr: int, data: np.ndarray, *, offsets: Optional[np.ndarray] = None):
        src = np.asarray(data).reshape(-1)
        if self._space is not None:
            sp = self._space
            if offsets is not None:
                idx = np.asarray(offsets, dtype=np.int64)
                n = int(idx.max()) + 1 if idx.size else 0
                flat = self._device_bytes(ptr, n * src.itemsize).view(src.dtype).copy()
                flat[idx] = src
            else:
                flat = src
                self._device_bytes(ptr, src.nbytes)          # bounds check
            sp.buf.upload(np.ascontiguousarray(flat).view(np.uint8), self.core_id * sp.bytes_per_core + ptr)
            return
        hit = self._find_staged(ptr)
        if hit is None:
            if offsets is not None:
                raise ValueError(f"Scatter to unmapped address 0x{ptr:x}")
            self._staged[ptr] = src.copy()
            return
        base, arr = hit
        DeviceHBM._put(arr, (ptr - base) // src.itemsize, src, offsets)

    def clear(self):
        self._staged.clear()
        self.next_ptr = 0
        self.used = 0
        if self._space is not None:
            sp = self._space
            sp.buf.memset(0, self.core_id * sp.bytes_per_core, sp.bytes_per_core)


class _LXList:
    """The per-core scratchpads, made when first touched."""

    def __init__(self, num_cores: int, size_mb: int):
        self._n, self._mb = num_cores, size_mb
        self._made: Dict[int, DeviceLX] = {}
        self._space = None

    def __len__(self):
        return self._n

    def __getitem__(self, core_id: int) -> DeviceLX:
        c = int(core_id)
        if c < 0:
            c += self._n
        if not 0 <= c < self._n:
            raise IndexError(f"core {core_id} out of range for {self._n} cores")
        if c not in self._made:
            self._made[c] = DeviceLX(c, self._mb)
            self._made[c].attach(self._space)
        return self._made[c]

    def __iter__(self):
        return (self[c] for c in range(self._n))

    def made(self) -> List[DeviceLX]:
        return [self._made[c] for c in sorted(self._made)]


class DeviceMemory:
    """``interp.memory`` (the reference's SpyreMemoryHierarchy,
    ``memory.py:449-463``): one HBM surface and one LX scratchpad per core."""

    def __init__(self, num_cores: int, lx_size_mb: int = 2):
        self.num_cores = num_cores
        self.lx_size_mb = lx_size_mb
        self.hbm = DeviceHBM()
        self.lx_scratchpads = _LXList(num_cores, lx_size_mb)

    def get_lx(self, core_id: int) -> DeviceLX:
        return self.lx_scratchpads[core_id]

    def lx_seeds(self) -> List[Tuple[int, int, np.ndarray]]:
        """(core, byte address, data) of everything staged in LX before the run."""
        return [(lx.core_id, addr, arr) for lx in self.lx_scratchpads.made() for addr, arr in lx.staged()]

    def attach_lx(self, space):
        for lx in self.lx_scratchpads.made():
            lx.attach(space)
        self.lx_scratchpads._space = space
