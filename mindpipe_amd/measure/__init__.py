"""Measurement-only read probes (``libmindpipe_measure.so``, built from ``probe.hip`` beside this
file).  Not part of the product path or its C ABI: ``bench.py --profile readfloor`` and
``--profile readsweep`` use them to measure what a launch that only reads costs on this GPU."""
from __future__ import annotations

import ctypes as C
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "libmindpipe_measure.so"
_LIB = None


def _load() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is not built (python -m mindpipe_amd.build)")
        lib = C.CDLL(str(LIB_PATH))
        lib.mp_probe_read_grid.restype = C.c_int64
        lib.mp_probe_read_grid.argtypes = [C.c_int64, C.c_int, C.c_int, C.c_int64]
        lib.mp_probe_read_shape.restype = C.c_int
        lib.mp_probe_read_shape.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_int64, C.c_void_p,
                                            C.c_void_p]
        lib.mp_probe_read_tiles.restype = C.c_int
        lib.mp_probe_read_tiles.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                            C.c_void_p]
        lib.mp_probe_cu_read.restype = C.c_int
        lib.mp_probe_cu_read.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                         C.c_void_p, C.c_void_p]
        lib.mp_probe_read_mfma_b.restype = C.c_int
        lib.mp_probe_read_mfma_b.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_int, C.c_int, C.c_void_p,
                                             C.c_void_p]
        _LIB = lib
    return _LIB


def probe_read(buf: torch.Tensor, sink: Optional[torch.Tensor] = None, threads: int = 256, loads: int = 4,
               grid: int = 0) -> torch.Tensor:
    """One launch that reads all of ``buf`` (contiguous, 16-byte multiple) and nothing else.
    ``grid`` = 0: one-shot workgroups of ``threads`` x ``loads`` 16-byte pieces (the one-row GEMVs'
    shape at the defaults); ``grid`` > 0: that many workgroups striding over the buffer.  Returns
    the sink the launch may write (pass it back in to reuse it)."""
    lib = _load()
    nbytes = buf.numel() * buf.element_size()
    if sink is None:
        words = max(1, int(lib.mp_probe_read_grid(nbytes, threads, loads, grid)))
        sink = torch.zeros(words, dtype=torch.int32, device=buf.device)
    rc = lib.mp_probe_read_shape(buf.data_ptr(), nbytes, threads, loads, grid, sink.data_ptr(),
                                 torch.cuda.current_stream(buf.device).cuda_stream)
    if rc != 0:
        raise RuntimeError(f"mp_probe_read_shape failed with status {rc}")
    return sink


def probe_read_tiles(buf: torch.Tensor, rows: int, row_bytes: int, tile_rows: int, step_bytes: int, depth: int,
                     sink: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One launch reading a row-major ``[rows, row_bytes]`` matrix in a tiled GEMM's weight order:
    a workgroup per ``tile_rows`` rows, ``step_bytes`` of each of its rows per step, ``depth`` steps
    in flight.  Returns the sink the launch may write."""
    lib = _load()
    if sink is None:
        sink = torch.zeros(max(1, -(-rows // tile_rows)), dtype=torch.int32, device=buf.device)
    rc = lib.mp_probe_read_tiles(buf.data_ptr(), rows, row_bytes, tile_rows, step_bytes, depth, sink.data_ptr(),
                                 torch.cuda.current_stream(buf.device).cuda_stream)
    if rc != 0:
        raise RuntimeError(f"mp_probe_read_tiles failed with status {rc}")
    return sink


def probe_cu_read(buf: torch.Tensor, region_bytes: int, nreg: int, passes: int, grid: int, threads: int = 256,
                  loads: int = 8, dma: bool = False, sink: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One launch of ``grid`` workgroups, workgroup w reading region ``w % nreg`` of ``buf``
    (``nreg`` regions of ``region_bytes``) ``passes`` times: the per-CU read rate from L2
    (``nreg`` = 8, one small region per XCD) or from HBM (large distinct regions).  ``dma``: the
    loads go straight to LDS.  Returns the sink the launch may write."""
    lib = _load()
    if buf.numel() * buf.element_size() < region_bytes * nreg:
        raise ValueError("buf is smaller than nreg regions")
    if sink is None:
        sink = torch.zeros(grid, dtype=torch.int32, device=buf.device)
    rc = lib.mp_probe_cu_read(buf.data_ptr(), region_bytes, nreg, passes, threads, loads, 1 if dma else 0, grid,
                              sink.data_ptr(), torch.cuda.current_stream(buf.device).cuda_stream)
    if rc != 0:
        raise RuntimeError(f"mp_probe_cu_read failed with status {rc}")
    return sink


def probe_read_mfma_b(buf: torch.Tensor, rows: int, row_bytes: int, kparts: int, depth: int,
                      sink: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One launch reading an int8 ``[rows, row_bytes]`` matrix in the lane order of an MFMA B operand
    loaded straight from memory (32 rows x 32 bytes per load instruction), ``kparts`` workgroups per 32
    rows splitting K, ``depth`` 128-byte K steps in flight.  Returns the sink the launch may write."""
    lib = _load()
    if sink is None:
        sink = torch.zeros(-(-rows // 32) * kparts, dtype=torch.int32, device=buf.device)
    rc = lib.mp_probe_read_mfma_b(buf.data_ptr(), rows, row_bytes, kparts, depth, sink.data_ptr(),
                                  torch.cuda.current_stream(buf.device).cuda_stream)
    if rc != 0:
        raise RuntimeError(f"mp_probe_read_mfma_b failed with status {rc}")
    return sink
