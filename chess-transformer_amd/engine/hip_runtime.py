"""The HIP runtime's entry points by address, for the native round loop: replaces the reference's engine/cuda_runtime.py.

The reference hands its Rust round loop (engine/selfplay_rs/src/rounds.rs:19-56) a table of libcudart function addresses
and calls a few of them from Python for its lean lanes (cuda_runtime.py:15-54). Here the table comes from
libchess_hip.so (chess_runtime_addresses), which is bound to the HIP runtime torch loaded, so the addresses are that
runtime's: hipSetDevice, hipMemcpyAsync, hipGraphLaunch, hipEventRecord, hipEventSynchronize, hipStreamSynchronize and
hipGetErrorString take the CUDA functions' arguments, and hipMemcpyKind's host-to-device (1) and device-to-host (2)
are CUDA's. addresses() gives them under the reference's key names, so the loop that reads them needs no change.
"""
from __future__ import annotations

import ctypes
import functools

import torch

from model.hip_kernels import load_library

HOST_TO_DEVICE, DEVICE_TO_HOST = 1, 2


class HipError(RuntimeError):
    pass


class HipRuntime:
    # in the order of chess_runtime_addresses; the waits release the GIL, the other calls return at once and keep it
    CALLS = {
        "cudaSetDevice": ([ctypes.c_int], False),
        "cudaMemcpyAsync": ([ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p], False),
        "cudaGraphLaunch": ([ctypes.c_void_p, ctypes.c_void_p], False),
        "cudaEventRecord": ([ctypes.c_void_p, ctypes.c_void_p], False),
        "cudaEventSynchronize": ([ctypes.c_void_p], True),
        "cudaStreamSynchronize": ([ctypes.c_void_p], True),
    }
    ERROR_STRING = "cudaGetErrorString"

    def __init__(self):
        torch.cuda.init()
        table = (ctypes.c_void_p * (len(self.CALLS) + 1))()
        library = load_library()
        if library.chess_runtime_addresses(table, len(table)) != 0:
            raise HipError(library.chess_last_error().decode())
        self.table = {name: table[index] for index, name in enumerate([*self.CALLS, self.ERROR_STRING])}
        calls = {}
        for name, (arguments, waits) in self.CALLS.items():
            kind = ctypes.CFUNCTYPE if waits else ctypes.PYFUNCTYPE
            calls[name] = kind(ctypes.c_int, *arguments)(self.table[name])
        self.error_string = ctypes.CFUNCTYPE(ctypes.c_char_p, ctypes.c_int)(self.table[self.ERROR_STRING])
        self.set_device, self.memcpy, self.graph_launch = calls["cudaSetDevice"], calls["cudaMemcpyAsync"], calls["cudaGraphLaunch"]
        self.event_record = calls["cudaEventRecord"]
        self.event_synchronize, self.stream_synchronize = calls["cudaEventSynchronize"], calls["cudaStreamSynchronize"]

    def check(self, error: int, what: str) -> None:
        if error:
            raise HipError(f"{what}: hip error {error}, {self.error_string(error).decode()}")

    def addresses(self) -> dict[str, int]:
        return dict(self.table)


@functools.cache
def hip_runtime() -> HipRuntime:
    return HipRuntime()


cuda_runtime = hip_runtime
CudaError = HipError
