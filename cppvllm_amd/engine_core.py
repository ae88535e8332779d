"""ctypes binding of the host serving core (``include/cppvllm_engine.h``, ``libcvh_engine.so``).

``EngineCore`` mirrors the reference's Scheduler/BlockManager surface (engine/scheduler.h,
engine/block_manager.h) as the model runner uses it: ``add_request``, ``schedule`` (a flat
ragged batch ordered by step group), ``postprocess`` (sampled tokens), ``is_finished``.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libcvh_engine.so"

CVE_OK, CVE_ERR_INVALID_ARG, CVE_ERR_TOO_LONG, CVE_ERR_STATE, CVE_ERR_EMPTY, CVE_ERR_BUSY = 0, -1, -2, -3, -4, -5
GROUP_DECODE, GROUP_FRESH, GROUP_CONT = 0, 1, 2


class Config(C.Structure):
    _fields_ = [("max_num_batched_tokens", C.c_int64), ("max_num_seqs", C.c_int64), ("max_chunk_tokens", C.c_int64),
                ("block_size", C.c_int32), ("num_blocks", C.c_int32), ("graph_max_blocks", C.c_int32),
                ("eos_token_id", C.c_int32)]


class _Batch(C.Structure):
    _fields_ = [("num_seqs", C.c_int64), ("num_tokens", C.c_int64), ("table_width", C.c_int64),
                ("group_start", C.c_int64 * 4), ("tokens", C.POINTER(C.c_int64)),
                ("positions", C.POINTER(C.c_int64)), ("cu_seqlens", C.POINTER(C.c_int64)),
                ("kv_lens", C.POINTER(C.c_int64)), ("block_tables", C.POINTER(C.c_int64)),
                ("samples", C.POINTER(C.c_int8)), ("seq_ids", C.POINTER(C.c_int64)),
                ("feed_src", C.POINTER(C.c_int64)), ("shared_blocks", C.POINTER(C.c_int32))]


class Stats(C.Structure):
    _fields_ = [("steps", C.c_int64), ("tokens_scheduled", C.c_int64), ("tokens_sampled", C.c_int64),
                ("preemptions", C.c_int64), ("finished", C.c_int64), ("free_blocks", C.c_int64),
                ("prefix_hit_tokens", C.c_int64)]


_LIB = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    path = Path(os.environ.get("CVE_LIB", LIB_PATH))
    if not path.exists():
        raise RuntimeError(f"{path} is missing: build it with `python -m cppvllm_amd.build`")
    h = C.CDLL(str(path))
    vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int32
    sig = {
        "cve_create": (vp, [C.POINTER(Config)]),
        "cve_destroy": (None, [vp]),
        "cve_add_request": (i64, [vp, C.POINTER(i32), i64, i32, i32]),
        "cve_schedule": (C.c_int, [vp, C.POINTER(_Batch)]),
        "cve_postprocess": (C.c_int, [vp, C.POINTER(i64), i64]),
        "cve_is_finished": (C.c_int, [vp]),
        "cve_num_outstanding": (i64, [vp]),
        "cve_get_stats": (C.c_int, [vp, C.POINTER(Stats)]),
        "cve_num_finished": (i64, [vp]),
        "cve_finished_output": (i64, [vp, i64, C.POINTER(i64), C.POINTER(i32), i64]),
        "cve_clear_finished": (None, [vp]),
        "cve_block_ref_count": (i32, [vp, i32]),
        "cve_block_table": (i64, [vp, i64, C.POINTER(i32), i64]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(h, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = h
    return h


@dataclass
class Batch:
    """One scheduled step (copies of the engine's arrays). Rows are ordered by group:
    ``group_start[g]:group_start[g+1]`` (decode, fresh prefill, continuation)."""
    tokens: np.ndarray          # int64 [T]
    positions: np.ndarray       # int64 [T]
    cu_seqlens: np.ndarray      # int64 [S+1]
    kv_lens: np.ndarray         # int64 [S]
    block_tables: np.ndarray    # int64 [S, W]
    samples: np.ndarray         # bool [S]
    seq_ids: np.ndarray         # int64 [S]
    group_start: tuple
    feed_src: np.ndarray = None  # int64 [T]: row of the previous step's samples feeding a token, or -1
    shared_blocks: np.ndarray = None  # int32 [S]: leading blocks other live sequences also reference

    @property
    def num_seqs(self) -> int:
        return len(self.kv_lens)

    @property
    def num_tokens(self) -> int:
        return len(self.tokens)


def _arr(ptr, n, dtype):
    if n == 0:
        return np.zeros(0, dtype=dtype)
    return np.ctypeslib.as_array(ptr, shape=(n,)).astype(dtype, copy=True)


class EngineBusy(RuntimeError):
    """Nothing can be scheduled until the oldest outstanding step is post-processed."""


class EngineCore:
    def __init__(self, *, max_num_batched_tokens=4096, max_num_seqs=256, max_chunk_tokens=1024, block_size=16,
                 num_blocks=1024, graph_max_blocks=256, eos_token_id=-1):
        self.cfg = Config(max_num_batched_tokens, max_num_seqs, max_chunk_tokens, block_size, num_blocks,
                          graph_max_blocks, eos_token_id)
        self._h = lib().cve_create(C.byref(self.cfg))
        if not self._h:
            raise ValueError("invalid engine configuration")

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h and _LIB is not None:
            _LIB.cve_destroy(h)

    def add_request(self, prompt, max_tokens: int, ignore_eos: bool = True) -> int:
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        rid = lib().cve_add_request(self._h, p.ctypes.data_as(C.POINTER(C.c_int32)), len(p), int(max_tokens),
                                    int(bool(ignore_eos)))
        if rid < 0:
            raise ValueError(f"add_request failed ({rid})")
        return rid

    def schedule(self) -> Batch | None:
        b = _Batch()
        code = lib().cve_schedule(self._h, C.byref(b))
        if code == CVE_ERR_BUSY:
            raise EngineBusy("retire the oldest step first")
        if code != CVE_OK:
            raise RuntimeError(f"schedule failed ({code})")
        if b.num_seqs == 0:
            return None
        S, T, W = b.num_seqs, b.num_tokens, b.table_width
        return Batch(tokens=_arr(b.tokens, T, np.int64), positions=_arr(b.positions, T, np.int64),
                     cu_seqlens=_arr(b.cu_seqlens, S + 1, np.int64), kv_lens=_arr(b.kv_lens, S, np.int64),
                     block_tables=_arr(b.block_tables, S * W, np.int64).reshape(S, W),
                     samples=_arr(b.samples, S, np.int8).astype(bool), seq_ids=_arr(b.seq_ids, S, np.int64),
                     group_start=tuple(int(x) for x in b.group_start), feed_src=_arr(b.feed_src, T, np.int64),
                     shared_blocks=_arr(b.shared_blocks, S, np.int32))

    def postprocess(self, sampled) -> None:
        s = np.ascontiguousarray(sampled, dtype=np.int64)
        code = lib().cve_postprocess(self._h, s.ctypes.data_as(C.POINTER(C.c_int64)), len(s))
        if code != CVE_OK:
            raise RuntimeError(f"postprocess failed ({code})")

    def is_finished(self) -> bool:
        return bool(lib().cve_is_finished(self._h))

    def outstanding(self) -> int:
        """Scheduled steps not yet post-processed (0..2)."""
        return int(lib().cve_num_outstanding(self._h))

    def stats(self) -> Stats:
        st = Stats()
        lib().cve_get_stats(self._h, C.byref(st))
        return st

    def take_finished(self) -> dict[int, list[int]]:
        out = {}
        n = lib().cve_num_finished(self._h)
        for i in range(n):
            rid = C.c_int64()
            cnt = lib().cve_finished_output(self._h, i, C.byref(rid), None, 0)
            buf = (C.c_int32 * max(cnt, 1))()
            lib().cve_finished_output(self._h, i, None, buf, cnt)
            out[rid.value] = list(buf[:cnt])
        lib().cve_clear_finished(self._h)
        return out

    def ref_count(self, block_id: int) -> int:
        return lib().cve_block_ref_count(self._h, block_id)

    def block_table(self, request_id: int) -> list[int] | None:
        n = lib().cve_block_table(self._h, request_id, None, 0)
        if n < 0:
            return None
        buf = (C.c_int32 * max(n, 1))()
        lib().cve_block_table(self._h, request_id, buf, n)
        return list(buf[:n])
