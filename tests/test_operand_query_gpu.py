"""Where the DMA kernels read an operand whose rows are not 16-byte aligned
in place, their 16-byte pieces reach up to 30 bytes past its last element.
hcg_operand_in_place reports the decision the GEMM entry points make; these
tests allocate device memory with known ends and launch no kernel.

* hipMalloc: an operand ending exactly at the end of its allocation must be
  copied (the bytes past it may be unmapped); one whose tail crosses a page
  boundary inside its allocation is read in place.
* Virtual memory management (an address range reserved larger than what is
  mapped, as allocators with expandable segments do): an operand ending at
  the end of the mapped part must be copied even though the reservation
  continues; inside the mapped part a page crossing is read in place.
"""

from __future__ import annotations

import ctypes

import pytest

from hc.gfx950 import _native

pytestmark = pytest.mark.gpu


def _hip():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    torch.cuda.init()
    return ctypes.CDLL("libamdhip64.so.7")  # the runtime torch already loaded


def _ok(rc: int, what: str) -> None:
    assert rc == 0, f"{what} returned {rc}"


def _ending_at(end: int, cols: int) -> int:
    """Base of a 1 x cols operand (cols odd: rows 2-byte aligned, not 16)
    whose last element ends exactly at ``end``."""
    assert cols % 2 == 1
    return end - 2 * cols


def test_hipmalloc_allocation_end_and_inner_page():
    hip = _hip()
    q = _native.load().hcg_operand_in_place
    size = 2 << 20
    ptr = ctypes.c_void_p()
    _ok(hip.hipMalloc(ctypes.byref(ptr), ctypes.c_size_t(size)), "hipMalloc")
    try:
        base = ptr.value
        cols = 1001
        at_end = _ending_at(base + size, cols)
        assert at_end % 16 != 0
        assert q(at_end, 1, cols, cols) == 0
        # the same operand ending 2 bytes before an inner page boundary
        inner = _ending_at(base + 4096 * 8 - 2, cols)
        assert q(inner, 1, cols, cols) == 1
        # two rows (row stride 1001 elements) ending at the allocation's end
        assert q(at_end - 2 * cols, 2, cols, cols) == 0
    finally:
        _ok(hip.hipFree(ptr), "hipFree")


class _MemLocation(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int), ("id", ctypes.c_int)]


class _AllocFlags(ctypes.Structure):
    _fields_ = [("compressionType", ctypes.c_ubyte), ("gpuDirectRDMACapable", ctypes.c_ubyte),
                ("usage", ctypes.c_ushort)]


class _AllocProp(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int), ("requestedHandleType", ctypes.c_int), ("location", _MemLocation),
                ("win32HandleMetaData", ctypes.c_void_p), ("allocFlags", _AllocFlags)]


class _AccessDesc(ctypes.Structure):
    _fields_ = [("location", _MemLocation), ("flags", ctypes.c_int)]


def test_reserved_range_larger_than_its_mapping():
    hip = _hip()
    q = _native.load().hcg_operand_in_place
    dev = ctypes.c_int()
    _ok(hip.hipGetDevice(ctypes.byref(dev)), "hipGetDevice")
    prop = _AllocProp(type=1, requestedHandleType=0, location=_MemLocation(type=1, id=dev.value))
    gran = ctypes.c_size_t()
    _ok(hip.hipMemGetAllocationGranularity(ctypes.byref(gran), ctypes.byref(prop), 0), "granularity")
    g = max(gran.value, 1 << 16)
    g = (g + gran.value - 1) // gran.value * gran.value
    handle = ctypes.c_void_p()
    _ok(hip.hipMemCreate(ctypes.byref(handle), ctypes.c_size_t(g), ctypes.byref(prop), ctypes.c_ulonglong(0)),
        "hipMemCreate")
    reserved = ctypes.c_void_p()
    mapped = False
    try:
        _ok(hip.hipMemAddressReserve(ctypes.byref(reserved), ctypes.c_size_t(3 * g), ctypes.c_size_t(0),
                                     None, ctypes.c_ulonglong(0)), "hipMemAddressReserve")
        _ok(hip.hipMemMap(reserved, ctypes.c_size_t(g), ctypes.c_size_t(0), handle, ctypes.c_ulonglong(0)),
            "hipMemMap")
        mapped = True
        desc = _AccessDesc(location=_MemLocation(type=1, id=dev.value), flags=3)
        _ok(hip.hipMemSetAccess(reserved, ctypes.c_size_t(g), ctypes.byref(desc), ctypes.c_size_t(1)),
            "hipMemSetAccess")
        base = reserved.value
        cols = 1001
        assert q(_ending_at(base + g, cols), 1, cols, cols) == 0
        assert q(_ending_at(base + 4096 * 4 - 2, cols), 1, cols, cols) == 1
    finally:
        if mapped:
            _ok(hip.hipMemUnmap(reserved, ctypes.c_size_t(g)), "hipMemUnmap")
        if reserved.value:
            _ok(hip.hipMemAddressFree(reserved, ctypes.c_size_t(3 * g)), "hipMemAddressFree")
        _ok(hip.hipMemRelease(handle), "hipMemRelease")
