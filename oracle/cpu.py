"""ctypes wrapper of the C oracle ``oracle/_build/libgdn_oracle.so``.

TEST INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke() checker, bench.py
cpu_baseline leg).  Takes numpy arrays in the layouts of include/gdn.h and
returns numpy results.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

LIB = Path(__file__).resolve().parent / "_build" / "libgdn_oracle.so"
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            from . import build as _b
            _b.build()
        h = ctypes.CDLL(str(LIB))
        vp, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        for name in ("gdn_cpu_recurrent_fwd", "gdn_cpu_chunk_fwd"):
            fn = getattr(h, name)
            fn.restype = i
            fn.argtypes = [vp] * 9 + [i] * 7 + [f, i, i]
        h.gdn_cpu_max_threads.restype = i
        _lib = h
    return _lib


def default_threads() -> int:
    """Thread count for checker runs in tests (OMP_NUM_THREADS, else at most 16)."""
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        return max(1, int(env))
    return max(1, min(16, os.cpu_count() or 1))


def host_threads() -> int:
    """Every core this process may run on (the timed CPU baseline uses them all)."""
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:  # pragma: no cover - non-Linux
        return max(1, os.cpu_count() or 1)


def host_info(threads: int) -> dict:
    """The host facts a CPU-baseline record carries: nproc, the cores this
    process may use, physical cores, the /proc/cpuinfo model, the thread
    count used, and the compiler and flags of the timed library."""
    import subprocess

    from . import build as _b

    model, phys = None, set()
    try:
        pid = core = None
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key, val = key.strip(), val.strip()
                if key == "model name" and model is None:
                    model = val
                elif key == "physical id":
                    pid = val
                elif key == "core id":
                    core = val
                elif not key and pid is not None and core is not None:
                    phys.add((pid, core))
                    pid = core = None
        if pid is not None and core is not None:
            phys.add((pid, core))
    except OSError:
        pass
    try:
        gcc = subprocess.run(["gcc", "--version"], capture_output=True, text=True,
                             timeout=10).stdout.splitlines()[0]
    except (OSError, subprocess.SubprocessError, IndexError):
        gcc = "gcc (version unavailable)"
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        affinity = None
    return {"nproc": os.cpu_count(), "cores_available": affinity,
            "physical_cores": len(phys) or None, "cpu_model": model, "threads": threads,
            "compiler": gcc, "cflags": " ".join(_b.CFLAGS)}


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def run(kind, q, k, v, g, beta, scale=None, initial_state=None, cu_seqlens=None,
        use_qk_l2norm=False, output_final_state=True, threads=None):
    """kind = 'chunk' | 'recurrent'.  Returns (o [B,T,Hv,V], state or None)."""
    q, k, v, g, beta = (_f32(x) for x in (q, k, v, g, beta))
    B, T, Hqk, K = q.shape
    Hv, V = v.shape[2], v.shape[3]
    cu = None
    if cu_seqlens is not None:
        cu = np.ascontiguousarray(np.asarray(cu_seqlens).reshape(-1), dtype=np.int32)
        N = cu.size - 1
    else:
        N = B
    h0 = None if initial_state is None else _f32(initial_state)
    ht = np.zeros((N, Hv, K, V), np.float32) if output_final_state else None
    o = np.zeros((B, T, Hv, V), np.float32)
    if scale is None:
        scale = K ** -0.5
    fn = lib().gdn_cpu_chunk_fwd if kind == "chunk" else lib().gdn_cpu_recurrent_fwd
    p = lambda a: None if a is None else a.ctypes.data  # noqa: E731
    rc = fn(p(q), p(k), p(v), p(g), p(beta), p(h0), p(ht), p(o), p(cu),
            B, T, Hqk, Hv, K, V, N, float(scale), int(bool(use_qk_l2norm)),
            int(threads or default_threads()))
    if rc != 0:
        raise ValueError(f"oracle {kind} rejected the arguments (rc={rc})")
    return o, ht
