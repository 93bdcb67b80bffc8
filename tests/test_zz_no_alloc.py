"""The allocation-free decode step (nie_paged_decode_append_noalloc) against
nie_paged_decode_append with a caller workspace, both called through the C ABI.

The caches and outputs must be bit-identical.  Calls in a row share the
library's static scratch: the second, smaller call reads partials written
over the first call's stale ones, and the third (4 short sequences, small
enough that with the one-pass rounding of fp32 its splits merge inside the
decode kernel) counts on the scratch's control region, which every call
leaves zero.  A call whose partials would not fit the scratch is rejected
with NIE_EINVAL before anything is launched.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from nano_infer_engine import _native, workloads

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
NIE_EINVAL = -1


def _log(msg: str) -> None:
    print(msg, flush=True)


def _same_bits(a: torch.Tensor, b: torch.Tensor) -> bool:
    ints = {torch.bfloat16: torch.int16, torch.float32: torch.int32}[a.dtype]
    return a.dtype == b.dtype and torch.equal(a.cpu().view(ints), b.cpu().view(ints))


def _host_lens(lens, host_plan):
    if not host_plan:
        return None, None
    arr = np.ascontiguousarray(np.asarray(lens, dtype=np.int32))
    return arr, arr.ctypes.data


def _call(lib, noalloc: bool, dtype, q, k_new, v_new, kc, vc, tables, lens_dev, lens, out, host_ptr):
    """One fused append + decode call on layer 0 through the C ABI."""
    num_layers, num_blocks, block_size, kv_heads, head_dim = kc.shape
    batch, q_heads, _ = q.shape
    code = _native.dtype_code(dtype)
    stream = torch.cuda.current_stream(DEV).cuda_stream
    common = (
        code, q.data_ptr(), q.stride(0), q.stride(1),
        k_new.data_ptr(), k_new.stride(0), v_new.data_ptr(), v_new.stride(0),
        None, None, 0,
        kc.data_ptr(), vc.data_ptr(), num_layers, 0, num_blocks, block_size,
        q_heads, kv_heads, head_dim,
        tables.data_ptr(), tables.shape[1],
        lens_dev.data_ptr(), batch, max(lens), sum(lens),
        ctypes.c_float(head_dim**-0.5),
        out.data_ptr(), out.stride(0), out.stride(1),
    )
    if noalloc:
        return lib.nie_paged_decode_append_noalloc(*common, host_ptr, stream)
    ws_bytes = lib.nie_paged_decode_workspace_bytes(code, batch, q_heads, kv_heads, head_dim, block_size, max(lens),
                                                    sum(lens), host_ptr)
    ws = torch.zeros(max(ws_bytes, 16), dtype=torch.uint8, device=DEV)  # the control region starts zeroed
    rc = lib.nie_paged_decode_append(*common, ws.data_ptr(), ws.numel(), host_ptr, stream)
    torch.cuda.synchronize()
    return rc


def _pair(lib, wl, dtype, host_plan):
    """(no-alloc cache K, V, out), (workspace cache K, V, out) for one workload."""
    kc, vc = wl.pool(dtype)
    q, k_new, v_new = wl.new_tokens(dtype)
    tables = torch.from_numpy(wl.table_array()).to(DEV)
    lens = list(wl.seq_lens)
    lens_dev = torch.tensor(lens, dtype=torch.int32, device=DEV)
    dq, dk, dv = q.to(DEV), k_new.to(DEV), v_new.to(DEV)
    results = []
    for noalloc in (True, False):
        k1, v1 = kc.to(DEV), vc.to(DEV)
        out = torch.empty(q.shape, dtype=dtype, device=DEV)
        arr, host_ptr = _host_lens(lens, host_plan)  # arr keeps the host copy alive over the call
        rc = _call(lib, noalloc, dtype, dq, dk, dv, k1, v1, tables, lens_dev, lens, out, host_ptr)
        torch.cuda.synchronize()
        assert rc == 0, lib.nie_last_error().decode()
        results.append((k1, v1, out))
        del arr
    return results


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("host_plan", [False, True])
def test_noalloc_matches_workspace_entry_point_twice(dtype, host_plan):
    lib = _native.load_library()
    assert lib.nie_paged_decode_noalloc_max_bytes() == 32 << 20
    # first call: the 16-sequence lognormal step (every long sequence split);
    # second call: 5 shorter sequences, still split, over the first call's
    # stale partials
    first = workloads.decode_ragged()
    second = workloads.ragged([40, 700, 1500, 3000, 5], [1] * 5, seed=21, pool_factor=1.5)
    third = workloads.decode_small()
    for name, wl in (("lognormal x16", first), ("ragged x5", second), ("small x4", third)):
        _log(f"noalloc {name} {dtype} host_plan={host_plan}")
        (ka, va, oa), (kb, vb, ob) = _pair(lib, wl, dtype, host_plan)
        assert _same_bits(ka, kb) and _same_bits(va, vb), f"{name}: cache differs"
        assert _same_bits(oa, ob), f"{name}: output differs"


def test_noalloc_rejects_calls_beyond_the_scratch():
    """2048 sequences of 4096 tokens need about 52 MB of split partials."""
    lib = _native.load_library()
    batch, lens = 2048, [4096] * 2048
    kc = torch.zeros((1, 16, 16, 8, 64), dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    q = torch.zeros((batch, 32, 64), dtype=torch.bfloat16, device=DEV)
    k_new = torch.zeros((batch, 8, 64), dtype=torch.bfloat16, device=DEV)
    v_new = torch.zeros_like(k_new)
    tables = torch.zeros((batch, 256), dtype=torch.int32, device=DEV)
    lens_dev = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = torch.empty_like(q)
    need = lib.nie_paged_decode_workspace_bytes(1, batch, 32, 8, 64, 16, 4096, sum(lens), None)
    assert need > lib.nie_paged_decode_noalloc_max_bytes()
    rc = _call(lib, True, torch.bfloat16, q, k_new, v_new, kc, vc, tables, lens_dev, lens, out, None)
    torch.cuda.synchronize()
    assert rc == NIE_EINVAL
    assert "static scratch" in lib.nie_last_error().decode()
