"""Build and load the gfx950 HIP library behind the PECO C-ABI (ctypes, no torch C++ ABI).

One shared library, ``peco_amd/_lib/libpeco_hip.so``, is compiled in-tree by hipcc from
``peco_amd/csrc/*.hip`` for ``--offload-arch=gfx950``. Every kernel launch goes to the
caller's stream (torch's current stream), and every tensor a native call touches is
retained with ``record_stream`` because the caching allocator cannot see ctypes accesses
(the reference does the same: peco/clustering_cuda.py:83-90, peco/attention_cuda.py:141-144).

There is no fallback: if the library is missing and cannot be built, calls raise.
"""
from __future__ import annotations

import ctypes
import fcntl
import os
import shutil
import subprocess
import threading
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
LIB_DIR = PACKAGE / "_lib"
LIB_PATH = Path(os.environ.get("PECO_HIP_LIBRARY", LIB_DIR / "libpeco_hip.so"))
ARCH = os.environ.get("PECO_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC",
    # Exact fp32: no implicit FMA contraction, correctly rounded division.
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    # Packed fp32 instructions are kept out of generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]

_LOCK = threading.Lock()
_LIB = None


def _hipcc() -> str:
    cand = os.environ.get("HIPCC")
    if cand:
        return cand
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    if path.exists():
        return str(path)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc is required to build the PECO HIP library")
    return found


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _stale() -> bool:
    if not LIB_PATH.exists():
        return True
    built = LIB_PATH.stat().st_mtime_ns
    deps = list(CSRC.glob("*.hip")) + list(CSRC.glob("*.hpp"))
    return any(p.stat().st_mtime_ns > built for p in deps)


def build_library(force: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libpeco_hip.so (atomic replace)."""
    LIB_DIR.mkdir(exist_ok=True)
    lock_path = LIB_DIR / ".build.lock"
    with open(lock_path, "w") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        if not force and not _stale():
            return LIB_PATH
        hipcc = _hipcc()
        obj_dir = LIB_DIR / "obj"
        obj_dir.mkdir(exist_ok=True)

        def compile_one(src: Path) -> Path:
            obj = obj_dir / (src.stem + ".o")
            cmd = [hipcc, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
            res = subprocess.run(cmd, capture_output=True, text=True)
            if res.returncode != 0:
                raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
            return obj

        srcs = sources()
        with ThreadPoolExecutor(max_workers=jobs or min(8, len(srcs))) as pool:
            objs = list(pool.map(compile_one, srcs))
        tmp = LIB_PATH.with_suffix(f".{os.getpid()}.tmp")
        cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link of {LIB_PATH.name} failed:\n{res.stderr}")
        os.replace(tmp, LIB_PATH)
    return LIB_PATH


P, I, Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
PP = ctypes.POINTER(ctypes.c_void_p)
IP = ctypes.POINTER(ctypes.c_int)

# name -> (restype, argtypes); mirrors include/peco_hip.h.
SIGNATURES = {
    # Reference ABI (peco/kernels/kmeans.cu:139,179,200,220; sparse_attention.cu:210,232).
    "peco_assign_tokens_to_centers": (I, [P] * 5 + [I] * 5 + [P]),
    "peco_recompute_cluster_centers": (I, [P] * 6 + [I] * 4 + [P]),
    "peco_reorder_token_features": (I, [P] * 3 + [I] * 5 + [P]),
    "peco_cluster_error_message": (ctypes.c_char_p, [I]),
    "peco_sparse_attention": (I, [P] * 8 + [I] * 7 + [P]),
    "peco_attention_error_string": (ctypes.c_char_p, [I]),
    # Extensions of the ABI.
    "peco_abi_version": (I, []),
    "peco_cluster_sort_workspace_size": (Z, [I, I, I]),
    "peco_cluster_sort": (I, [P, I, I, I, P, P, P, P, P, Z, P]),
    "peco_kmeans_workspace_size": (Z, [I, I, I, I]),
    "peco_kmeans_fit": (I, [I, PP, P, PP, PP, PP, PP, PP, PP, IP, IP, IP, I, I, I, P, Z, P]),
    "peco_kmeans_screen": (I, [P, I, P, P, P, P, I, I, I, I, P]),
    "peco_kmeans_screen_bound": (None, [I, P, P]),
    "peco_base_offset_encode": (I, [P, I, P, P, I, I, I, I, I, P, P, P, P]),
    "peco_base_offset_decode": (I, [P, P, P, P, P, I, I, I, I, I, P, P]),
    "peco_base_offset_fake_quant": (I, [P, I, P, P, I, I, I, I, I, P, P]),
    "peco_pack_clustered": (I, [PP, PP, PP, PP, PP, IP, IP, I, I, I, I, I, I, P]),
    "peco_sparse_attention_workspace_size": (Z, [I, I, I, I, I]),
    "peco_sparse_attention_ex": (I, [P] * 8 + [I, P, P, Z] + [I] * 7 + [P]),
    "peco_sparse_attention_indexed": (I, [P] * 9 + [I, P, P, Z] + [I] * 7 + [P]),
    "peco_select_cluster_connections": (I, [P] * 4 + [I] * 4 + [ctypes.c_float] + [I] * 4 + [P] * 5),
    "peco_sparse_attention_noalloc": (I, [P] * 7 + [I] * 7 + [P]),
    "peco_kmeans_fit_pack": (I, [I, PP, P, PP, PP, PP, PP, PP, PP, IP, IP, IP, I, I, I, PP, IP, PP, PP, PP, PP, PP, I, I,
                                 P, Z, P]),
    "peco_select_work_size": (Z, [I] * 5),
    "peco_select_work": (I, [P] * 4 + [I] * 4 + [ctypes.c_float] + [I] * 6 + [P] * 4 + [Z, P]),
    "peco_sparse_attention_work": (I, [P] * 5 + [I, P, P, I, I, P, Z] + [I] * 7 + [P]),
    "peco_base_offset_attention": (I, [P, P, P, I] + [P] * 9 + [I, I] + [P] * 5 + [Z] + [I] * 8 + [P]),
}


def library() -> ctypes.CDLL:
    """Load the HIP library once (building it first if it was never built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        if not LIB_PATH.exists():
            build_library()
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
        return lib


def check(status: int, what: str) -> None:
    if status:
        msg = library().peco_cluster_error_message(status).decode("utf-8", errors="replace")
        raise RuntimeError(f"{what} failed: {msg} (status {status})")


def ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def ptr_array(tensors) -> ctypes.Array:
    return (ctypes.c_void_p * len(tensors))(*[(t.data_ptr() if t is not None else 0) for t in tensors])


def int_array(values) -> ctypes.Array:
    return (ctypes.c_int * len(values))(*values)


def current_stream(device, *tensors) -> ctypes.c_void_p:
    """Record every tensor on the current stream and return that stream's handle."""
    import torch

    stream = torch.cuda.current_stream(device)
    for t in tensors:
        if t is not None:
            t.record_stream(stream)
    return ctypes.c_void_p(stream.cuda_stream)


# hipEventDisableSystemFence (hip_runtime_api.h): the event skips the system-scope cache writeback
# and invalidation of a default event when it is recorded.
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000


class _HipEvents:
    """hipEventCreateWithFlags / Record / ElapsedTime / Destroy, resolved through this library's
    own dependency on the HIP runtime (the one torch has loaded)."""

    def __init__(self):
        lib = library()
        self.create = lib.hipEventCreateWithFlags
        self.create.argtypes, self.create.restype = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint], ctypes.c_int
        self.record = lib.hipEventRecord
        self.record.argtypes, self.record.restype = [ctypes.c_void_p, ctypes.c_void_p], ctypes.c_int
        self.elapsed = lib.hipEventElapsedTime
        self.elapsed.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.elapsed.restype = ctypes.c_int
        self.destroy = lib.hipEventDestroy
        self.destroy.argtypes, self.destroy.restype = [ctypes.c_void_p], ctypes.c_int


_HIP_EVENTS = None


class FencelessEvent:
    """A HIP timing event created with hipEventDisableSystemFence, with the record/elapsed_time
    interface of torch.cuda.Event. The HIP runtime documents the flag for events used only to
    measure time: recording one performs no system-scope cache writeback and invalidation, so it
    perturbs the work it times less than a default event does. Read it after a synchronize."""

    def __init__(self):
        global _HIP_EVENTS
        if _HIP_EVENTS is None:
            _HIP_EVENTS = _HipEvents()
        self._api = _HIP_EVENTS
        self._event = ctypes.c_void_p()
        if self._api.create(ctypes.byref(self._event), HIP_EVENT_DISABLE_SYSTEM_FENCE) != 0:
            raise RuntimeError("hipEventCreateWithFlags failed")

    def record(self, stream=None):
        """Record on `stream` (a hipStream_t), by default torch's current stream."""
        if stream is None:
            import torch

            stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        if self._api.record(self._event, stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_time(self, end):
        ms = ctypes.c_float()
        if self._api.elapsed(ctypes.byref(ms), self._event, end._event) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def __del__(self):
        if getattr(self, "_event", None) and self._event.value:
            self._api.destroy(self._event)


class LaunchTimer:
    """FencelessEvent pairs recorded immediately around kernel launches, for measurement:
    start(stream) and stop(stream) around each launch, then elapsed_ms() after a synchronize."""

    def __init__(self):
        self._pairs = []
        self._open = None

    def start(self, stream):
        self._open = FencelessEvent()
        self._open.record(stream)

    def stop(self, stream):
        end = FencelessEvent()
        end.record(stream)
        self._pairs.append((self._open, end))
        self._open = None

    def __len__(self):
        return len(self._pairs)

    def elapsed_ms(self):
        """The recorded pairs' durations in ms (the events are released)."""
        out = [start.elapsed_time(end) for start, end in self._pairs]
        self._pairs = []
        return out


DTYPE_CODES = {}


def dtype_code(dtype) -> int:
    import torch

    if not DTYPE_CODES:
        DTYPE_CODES.update({torch.float16: 0, torch.bfloat16: 1, torch.float32: 2})
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}") from None
