"""ctypes binding of libpkhost.so (include/pkhost.h) and the Python face of the host core.

HostScheduler owns the step buffers (pinned host memory when a GPU is present) that the
C++ core fills with the arrays of ModelRunner.prepare_seqs (src/engine/model_runner.py:
174-233), so one step's host work is one C call plus the host-to-device copies.
"""
from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

HOST_LIB_PATH = Path(__file__).resolve().with_name("libpkhost.so")

PKH_OK = 0
PKH_ERR_INVALID_ARG = -1
PKH_ERR_CAPACITY = -2
PKH_ERR_STATE = -3


class PkhConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "num_blocks", "block_size", "max_num_seqs", "max_num_batched_tokens",
        "chunked_prefill_size", "max_live_seqs", "eos")]


class PkhStep(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "num_seqs", "num_tokens", "num_prefill_tokens", "num_decode_tokens", "max_seqlen_q",
        "max_seqlen_k", "is_prefill", "block_table_width")] + [
        (n, ctypes.c_void_p) for n in (
            "input_ids", "positions", "cu_seqlens_q", "cu_seqlens_k", "slot_mapping",
            "context_lens", "block_tables", "seq_ids")]


_vp, _i32, _i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
SIGNATURES = {
    "pkh_last_error": (ctypes.c_char_p, []),
    "pkh_create": (_vp, [ctypes.POINTER(PkhConfig)]),
    "pkh_destroy": (None, [_vp]),
    "pkh_set_buffers": (ctypes.c_int, [_vp] + [_vp] * 8 + [_i32, _i32, _i32]),
    "pkh_add_request": (_i64, [_vp, _vp, _i32, _i32, _i32]),
    "pkh_schedule": (ctypes.c_int, [_vp, ctypes.POINTER(PkhStep)]),
    "pkh_postprocess": (ctypes.c_int, [_vp, _vp, _i32, ctypes.POINTER(_i32)]),
    "pkh_is_finished": (ctypes.c_int, [_vp]),
    "pkh_num_free_blocks": (_i32, [_vp]),
    "pkh_generated": (_i32, [_vp, _i64, _vp, _i32]),
    "pkh_num_generated": (_i32, [_vp, _i64]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def host_lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not HOST_LIB_PATH.exists():
                raise RuntimeError(f"{HOST_LIB_PATH.name} is not built; run `python -m pagedkv.build`")
            h = ctypes.CDLL(str(HOST_LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(h, name)
                fn.restype = res
                fn.argtypes = args
            _lib = h
    return _lib


class HostError(RuntimeError):
    pass


def _check(code: int, what: str) -> None:
    if code < 0:
        raise HostError(f"{what} failed with code {code}: {host_lib().pkh_last_error().decode()}")


@dataclass
class Step:
    """One step's batch: host tensors (views of the pinned buffers) and launch bounds."""
    num_seqs: int
    num_tokens: int
    num_prefill_tokens: int
    num_decode_tokens: int
    max_seqlen_q: int
    max_seqlen_k: int
    is_prefill: bool
    input_ids: torch.Tensor
    positions: torch.Tensor
    cu_seqlens_q: torch.Tensor
    cu_seqlens_k: torch.Tensor
    slot_mapping: torch.Tensor
    context_lens: torch.Tensor
    block_tables: torch.Tensor | None
    seq_ids: torch.Tensor


class HostScheduler:
    """Scheduler + block pool + context construction of the reference engine, in C++.

    Mirrors Scheduler (src/engine/scheduler.py), the allocation half of BlockManager
    (src/engine/block_manager.py:183-246) and ModelRunner.prepare_seqs
    (src/engine/model_runner.py:168-233); defaults follow RunnerConfig
    (src/config/runner_config.py:11-20) and the 128-sequence admission cap of
    scheduler.py:37.
    """

    def __init__(self, num_blocks: int, block_size: int = 256, max_num_seqs: int = 512,
                 max_num_batched_tokens: int = 16384, chunked_prefill_size: int = 512,
                 max_live_seqs: int = 128, eos: int = -1, max_seq_len: int = 8192,
                 pin_memory: bool | None = None):
        lib = host_lib()
        cfg = PkhConfig(num_blocks, block_size, max_num_seqs, max_num_batched_tokens,
                        chunked_prefill_size, max_live_seqs, eos)
        self._h = lib.pkh_create(ctypes.byref(cfg))
        if not self._h:
            raise HostError(lib.pkh_last_error().decode())
        self.block_size = block_size
        self.num_blocks = num_blocks
        pin = torch.cuda.is_available() if pin_memory is None else pin_memory
        width = (max_seq_len + block_size - 1) // block_size
        mk = lambda n, dt: torch.empty(n, dtype=dt, pin_memory=pin)  # noqa: E731
        self._buf = dict(
            input_ids=mk(max_num_batched_tokens, torch.int64),
            positions=mk(max_num_batched_tokens, torch.int64),
            cu_seqlens_q=mk(max_num_seqs + 1, torch.int32),
            cu_seqlens_k=mk(max_num_seqs + 1, torch.int32),
            slot_mapping=mk(max_num_batched_tokens, torch.int32),
            context_lens=mk(max_num_seqs, torch.int32),
            block_tables=mk(max_num_seqs * width, torch.int32),
            seq_ids=mk(max_num_seqs, torch.int64),
        )
        b = self._buf
        _check(lib.pkh_set_buffers(
            self._h, b["input_ids"].data_ptr(), b["positions"].data_ptr(),
            b["cu_seqlens_q"].data_ptr(), b["cu_seqlens_k"].data_ptr(),
            b["slot_mapping"].data_ptr(), b["context_lens"].data_ptr(),
            b["block_tables"].data_ptr(), b["seq_ids"].data_ptr(),
            max_num_batched_tokens, max_num_seqs, width), "pkh_set_buffers")
        self._step = PkhStep()
        self._tok = np.empty(max_num_seqs, dtype=np.int32)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            host_lib().pkh_destroy(h)
            self._h = None

    def add_request(self, prompt, max_tokens: int, ignore_eos: bool = False) -> int:
        arr = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32))
        sid = host_lib().pkh_add_request(self._h, arr.ctypes.data, arr.size, int(max_tokens),
                                         1 if ignore_eos else 0)
        if sid < 0:
            _check(int(sid), "add_request")
        return int(sid)

    def schedule(self) -> Step | None:
        """The next step's batch, or None when every sequence has finished."""
        st = self._step
        _check(host_lib().pkh_schedule(self._h, ctypes.byref(st)), "schedule")
        if st.num_seqs == 0:
            return None
        b, s, n = self._buf, st.num_seqs, st.num_tokens
        w = st.block_table_width
        return Step(
            num_seqs=s, num_tokens=n, num_prefill_tokens=st.num_prefill_tokens,
            num_decode_tokens=st.num_decode_tokens, max_seqlen_q=st.max_seqlen_q,
            max_seqlen_k=st.max_seqlen_k, is_prefill=bool(st.is_prefill),
            input_ids=b["input_ids"][:n], positions=b["positions"][:n],
            cu_seqlens_q=b["cu_seqlens_q"][:s + 1], cu_seqlens_k=b["cu_seqlens_k"][:s + 1],
            slot_mapping=b["slot_mapping"][:n], context_lens=b["context_lens"][:s],
            block_tables=b["block_tables"][:s * w].view(s, w) if w else None,
            seq_ids=b["seq_ids"][:s])

    def postprocess(self, token_ids) -> int:
        """Scheduler.postprocess with the step's sampled tokens (batch order)."""
        arr = np.ascontiguousarray(np.asarray(token_ids, dtype=np.int32))
        fin = ctypes.c_int32(0)
        _check(host_lib().pkh_postprocess(self._h, arr.ctypes.data, arr.size, ctypes.byref(fin)),
               "postprocess")
        return fin.value

    def is_finished(self) -> bool:
        return bool(host_lib().pkh_is_finished(self._h))

    def num_free_blocks(self) -> int:
        return int(host_lib().pkh_num_free_blocks(self._h))

    def generated(self, seq_id: int) -> list[int]:
        n = host_lib().pkh_num_generated(self._h, seq_id)
        _check(n, "num_generated")
        out = np.empty(max(n, 1), dtype=np.int32)
        got = host_lib().pkh_generated(self._h, seq_id, out.ctypes.data, n)
        _check(got, "generated")
        return out[:got].tolist()
