"""The allocation-free v2 entry point (``ayk_paged_attention_v2_static``), through the C ABI.

Its partials and arrival counters live in the library's static device array. Each call is
checked, bit for bit, against ``ayk_paged_attention_v2`` given a workspace and counters of
its own (the same kernels and launch), on two calls in a row whose second is smaller, for
either merge site and for a staged (graph-replay) split; a call whose partials exceed the
static array is refused before any launch.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from ayaka_amd.hip import _lib
from ayaka_amd.hip import attention as hip_attention
from oracle.numerics import parity_report
from tests._support import build_scenario

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
STATIC_PARTIAL_BYTES = 63 << 20  # AYK_V2_STATIC_SCRATCH_BYTES


def _device(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def _call(lib, static: bool, out, s, tensors, size: int, parts: int, work, n_work: int, staged, flags: int,
          scratch=None, arrivals=None) -> int:
    q, k, v, table, lengths = tensors
    width = table.shape[1]
    common = (out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr(), width,
              lengths.data_ptr(), None, None, len(s.lengths), s.heads, s.kv_heads, s.head_dim, k.shape[0],
              s.block_size, width, 0, 1, 1, ctypes.c_float(s.scale), 1.0, 1.0, size, parts, work, n_work, staged)
    stream = torch.cuda.current_stream().cuda_stream
    if static:
        return lib.ayk_paged_attention_v2_static(*common, flags, stream)
    return lib.ayk_paged_attention_v2(*common, scratch.data_ptr(), scratch.numel(), arrivals.data_ptr(), flags,
                                      stream)


def _static_counters(lib) -> torch.Tensor:
    """The static array's arrival counters on this device, viewed in place as int32."""
    ptr, words = ctypes.c_void_p(), ctypes.c_int64()
    assert lib.ayk_paged_attention_v2_static_counters(ctypes.byref(ptr), ctypes.byref(words)) == 0
    assert ptr.value and words.value == 1 << 18

    class _View:
        __cuda_array_interface__ = {"shape": (words.value,), "typestr": "<i4", "data": (ptr.value, False),
                                    "version": 3, "strides": None}

    return torch.as_tensor(_View(), device=DEV)


def _scenario(steps, heads: int, seed: int):
    s = build_scenario(steps, heads=heads, kv_heads=2, head_dim=128, block_size=16, mode="decode", seed=seed)
    table = torch.from_numpy(s.table.astype(np.int32)).to(DEV)
    lengths = torch.tensor(s.lengths, dtype=torch.int32, device=DEV)
    return s, (_device(s.q_bits), _device(s.k_bits), _device(s.v_bits), table, lengths)


@pytest.mark.parametrize("heads", [8, 4], ids=["mfma", "dpp"])
@pytest.mark.parametrize("flags", [0, 8, 16], ids=["library", "reduce-kernel", "in-kernel"])
def test_static_scratch_matches_the_workspace_entry_point(flags: int, heads: int) -> None:
    lib = _lib.lib()
    # the second call is smaller (fewer rows, shorter contexts) and follows the first on the
    # same static array: nothing of the first may leak into it
    for steps, size, seed in (([(1, 2100), (1, 1), (1, 0), (1, 900), (1, 1500), (1, 64)], 256, 81),
                              ([(1, 700), (1, 33)], 128, 82)):
        s, tensors = _scenario(steps, heads, seed)
        print(f"static v2: rows {len(s.lengths)} size {size} flags {flags} heads {heads}", flush=True)
        parts = -(-tensors[3].shape[1] * s.block_size // size)
        items = torch.from_numpy(hip_attention.work_list(s.lengths, size)).to(DEV)
        nbytes = lib.ayk_paged_attention_v2_workspace_bytes(len(s.lengths), heads, 128, parts)
        scratch = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        arrivals = torch.zeros(len(s.lengths) * heads, dtype=torch.int32, device=DEV)
        outs = []
        for static in (True, False, True):
            out = torch.full_like(tensors[0], float("nan"))
            rc = _call(lib, static, out, s, tensors, size, parts, items.data_ptr(), items.numel() // 2, None, flags,
                       scratch, arrivals)
            assert rc == 0, lib.ayk_last_error()
            torch.cuda.synchronize()
            outs.append(out)
        assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
        assert torch.equal(outs[2].view(torch.int16), outs[1].view(torch.int16))
        expected = s.expected(np.float64)
        got = outs[0].float().cpu().numpy()
        rep = parity_report(got, expected, "bf16")
        assert rep["max_abs_excess"] <= 2e-3 and rep["rel_l2"] <= 1e-3, rep
        assert int(arrivals.abs().sum()) == 0
        assert int(torch.count_nonzero(_static_counters(lib))) == 0


def test_static_counters_stay_zero_when_a_larger_call_follows() -> None:
    # the in-kernel merge counts finished partitions in the static array's counters; a call over
    # more (row, head) pairs than the one before it reads counters the earlier call never
    # touched, so each call must leave every counter at zero, read back from the array itself
    lib = _lib.lib()
    counters = _static_counters(lib)
    assert int(torch.count_nonzero(counters)) == 0
    for steps, size, seed in (([(1, 300), (1, 40)], 64, 85),
                              ([(1, 900), (1, 1), (1, 0), (1, 700), (1, 350)] * 3, 128, 86)):
        s, tensors = _scenario(steps, 8, seed)
        print(f"static v2 counters: rows {len(s.lengths)} size {size}", flush=True)
        parts = -(-tensors[3].shape[1] * s.block_size // size)
        items = torch.from_numpy(hip_attention.work_list(s.lengths, size)).to(DEV)
        nbytes = lib.ayk_paged_attention_v2_workspace_bytes(len(s.lengths), 8, 128, parts)
        scratch = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        arrivals = torch.zeros(len(s.lengths) * 8, dtype=torch.int32, device=DEV)
        outs = []
        for static in (True, False):
            out = torch.full_like(tensors[0], float("nan"))
            rc = _call(lib, static, out, s, tensors, size, parts, items.data_ptr(), items.numel() // 2, None, 16,
                       scratch, arrivals)
            assert rc == 0, lib.ayk_last_error()
            torch.cuda.synchronize()
            outs.append(out)
        assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
        assert int(torch.count_nonzero(counters)) == 0


def test_static_scratch_follows_a_staged_split() -> None:
    # as a graph replay calls it: split and work list read from device memory, partials packed
    lib = _lib.lib()
    for steps, size, seed in (([(1, 700), (1, 1), (1, 0), (1, 300)], 192, 83), ([(1, 90), (1, 5)], 64, 84)):
        s, tensors = _scenario(steps, 8, seed)
        n_rows, width = len(s.lengths), tensors[3].shape[1]
        parts = -(-width * 16 // 64)
        capacity = n_rows * parts
        items = hip_attention.work_list(s.lengths, size)
        counts = [-(-n // size) for n in s.lengths]
        staged = torch.tensor([size, items.size // 2, *[sum(counts[:r]) for r in range(n_rows)], *items.tolist()]
                              + [0] * (2 * capacity - items.size), dtype=torch.int32, device=DEV)
        work = staged.data_ptr() + 4 * (2 + n_rows)
        nbytes = lib.ayk_paged_attention_v2_workspace_bytes(capacity, 8, 128, 1)
        scratch = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        arrivals = torch.zeros(n_rows * 8, dtype=torch.int32, device=DEV)
        outs = []
        for static in (True, False):
            out = torch.full_like(tensors[0], float("nan"))
            rc = _call(lib, static, out, s, tensors, 64, parts, work, capacity, staged.data_ptr(), 0, scratch,
                       arrivals)
            assert rc == 0, lib.ayk_last_error()
            torch.cuda.synchronize()
            outs.append(out)
        assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def test_calls_beyond_the_static_scratch_are_refused() -> None:
    lib = _lib.lib()
    # 512 rows x 32 heads x 8 partitions x (128 + 2) floats = 68 MB of partials: refused, no launch
    assert lib.ayk_paged_attention_v2_workspace_bytes(512, 32, 128, 8) > STATIC_PARTIAL_BYTES
    rc = lib.ayk_paged_attention_v2_static(1, 1, 1, 1, 1, 8, 1, None, None, 512, 32, 8, 128, 100, 16, 8, 0, 1, 1,
                                           ctypes.c_float(1.0), 1.0, 1.0, 64, 8, None, 0, None, 0, None)
    assert rc == 4 and b"static scratch" in lib.ayk_last_error()
