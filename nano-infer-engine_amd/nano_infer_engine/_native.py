"""ctypes binding of ``libnie_hip.so``, the gfx950 paged-attention library.

Every function here takes torch tensors that live on a ROCm device, checks
them, and calls one C entry point declared in ``include/nie_paged.h`` on the
current HIP stream of that device.  There is no CPU path: a tensor on
another device, or a missing library, raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import os
import threading

import numpy as np
import torch

LIBRARY_NAME = "libnie_hip.so"

NIE_DTYPE_F32 = 0
NIE_DTYPE_BF16 = 1

#: Rounding points of the bf16 attention probabilities (``set_attention_rounding``).
NIE_ROUND_REFERENCE = 0
NIE_ROUND_FAST = 1
ROUNDING_MODES = {"reference": NIE_ROUND_REFERENCE, "fast": NIE_ROUND_FAST}

_DTYPE_CODES = {torch.float32: NIE_DTYPE_F32, torch.bfloat16: NIE_DTYPE_BF16}

#: Head dims and GQA group sizes the attention kernels are built for.
#: Shapes the MFMA decode / prefill kernels are built for ("tuned"); every
#: other head_dim up to GENERIC_MAX_HEAD_DIM and every GQA group runs on the
#: library's generic attention kernel (same results, far lower rate).
SUPPORTED_HEAD_DIMS = (64, 128)
SUPPORTED_GROUP_SIZES = (1, 2, 4, 8, 16)
GENERIC_MAX_HEAD_DIM = 256


def tuned_attention(q_heads: int, kv_heads: int, head_dim: int) -> bool:
    """Whether the shape runs on the MFMA kernels (which need 16-byte aligned rows)."""
    return head_dim in SUPPORTED_HEAD_DIMS and q_heads % kv_heads == 0 and q_heads // kv_heads in SUPPORTED_GROUP_SIZES


def _row_align(q_heads: int, kv_heads: int, head_dim: int) -> int:
    """Byte alignment the launch needs of its row pointers and strides."""
    return 16 if tuned_attention(q_heads, kv_heads, head_dim) else 1

#: Every symbol the library exports (checked by the CPU test suite).
EXPORTED_SYMBOLS = (
    "nie_version",
    "nie_last_error",
    "nie_kv_append",
    "nie_kv_gather",
    "nie_kv_copy_blocks",
    "nie_rope_kv_append",
    "nie_argmax_rows",
    "nie_argmax_rows_workspace_bytes",
    "nie_argmax_rows_split",
    "nie_rms_norm",
    "nie_silu_mul",
    "nie_linear_rows",
    "nie_rms_norm_linear_rows",
    "nie_set_attention_rounding",
    "nie_attention_rounding",
    "nie_set_decode_fused",
    "nie_decode_fused",
    "nie_set_decode_fused_spin",
    "nie_workspace_control_bytes",
    "nie_decode_last_path",
    "nie_paged_decode_workspace_bytes",
    "nie_paged_decode",
    "nie_paged_decode_append",
    "nie_paged_decode_plan_bytes",
    "nie_paged_decode_plan",
    "nie_paged_decode_append_planned",
    "nie_paged_decode_noalloc_max_bytes",
    "nie_paged_decode_append_noalloc",
    "nie_varlen_prefill_workspace_bytes",
    "nie_varlen_prefill",
)

_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p
_f32 = ctypes.c_float

_SIGNATURES = {
    "nie_version": (ctypes.c_char_p, []),
    "nie_last_error": (ctypes.c_char_p, []),
    "nie_kv_append": (
        _i32,
        [_i32, _ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _i64, _ptr],
    ),
    "nie_kv_gather": (
        _i32,
        [_i32, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _ptr],
    ),
    "nie_kv_copy_blocks": (
        _i32,
        [_i32, _ptr, _ptr, _i64, _ptr, _ptr, _ptr, _i64, _ptr, _i64, _i64, _i64, _i64, _i64, _ptr],
    ),
    "nie_rope_kv_append": (
        _i32,
        [
            _i32, _ptr, _i64, _i64, _i64,    # dtype, q, q strides, q_heads
            _ptr, _i64, _i64,                # k, strides
            _ptr, _i64, _i64,                # v, strides
            _ptr, _ptr, _i64,                # positions, slots, tokens
            _ptr, _ptr, _i64,                # cos, sin, table rows
            _ptr, _ptr,                      # caches
            _i64, _i64, _i64, _i64,          # layers, layer, blocks, block_size
            _i64, _i64, _ptr,                # kv_heads, head_dim, stream
        ],
    ),
    "nie_argmax_rows": (_i32, [_i32, _ptr, _i64, _i64, _i64, _ptr, _ptr]),
    "nie_argmax_rows_workspace_bytes": (_i64, [_i64, _i64]),
    "nie_argmax_rows_split": (_i32, [_i32, _ptr, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr]),
    "nie_rms_norm": (
        _i32,
        [_i32, _ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, _f32, _ptr],
    ),
    "nie_silu_mul": (_i32, [_i32, _ptr, _i64, _ptr, _i64, _ptr, _i64, _i64, _i64, _ptr]),
    "nie_linear_rows": (_i32, [_i32, _ptr, _i64, _i64, _ptr, _i64, _i64, _i32, _ptr, _i64, _ptr]),
    "nie_rms_norm_linear_rows": (
        _i32,
        [_i32, _ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr, _f32, _i64, _ptr, _i64, _i64, _i32, _ptr, _i64, _ptr],
    ),
    "nie_set_attention_rounding": (_i32, [_i32]),
    "nie_attention_rounding": (_i32, []),
    "nie_set_decode_fused": (_i32, [_i32]),
    "nie_decode_fused": (_i32, []),
    "nie_set_decode_fused_spin": (_i32, [_i32]),
    "nie_workspace_control_bytes": (_i64, []),
    "nie_decode_last_path": (_i32, []),
    "nie_paged_decode_workspace_bytes": (_i64, [_i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _ptr]),
    "nie_paged_decode": (
        _i32,
        [
            _i32, _ptr, _i64, _i64,          # dtype, q, q strides
            _ptr, _ptr,                      # caches
            _i64, _i64, _i64, _i64,          # layers, layer, blocks, block_size
            _i64, _i64, _i64,                # q_heads, kv_heads, head_dim
            _ptr, _i64,                      # block tables, stride
            _ptr, _i64, _i64, _i64,          # seq_lens, batch, max, total
            _f32,                            # scale
            _ptr, _i64, _i64,                # out, strides
            _ptr, _i64,                      # workspace, bytes
            _ptr, _ptr,                      # host seq_lens, stream
        ],
    ),
    "nie_paged_decode_append": (
        _i32,
        [
            _i32, _ptr, _i64, _i64,          # dtype, q, q strides
            _ptr, _i64, _ptr, _i64,          # new K rows, stride, new V rows, stride
            _ptr, _ptr, _i64,                # RoPE cos / sin tables, rows
            _ptr, _ptr,                      # caches
            _i64, _i64, _i64, _i64,          # layers, layer, blocks, block_size
            _i64, _i64, _i64,                # q_heads, kv_heads, head_dim
            _ptr, _i64,                      # block tables, stride
            _ptr, _i64, _i64, _i64,          # seq_lens, batch, max, total
            _f32,                            # scale
            _ptr, _i64, _i64,                # out, strides
            _ptr, _i64,                      # workspace, bytes
            _ptr, _ptr,                      # host seq_lens, stream
        ],
    ),
    "nie_paged_decode_plan_bytes": (_i64, []),
    "nie_paged_decode_plan": (
        _i32,
        [
            _i32, _i64, _i64, _i64, _i64,    # dtype, q_heads, kv_heads, head_dim, block_size
            _ptr, _i64, _i64, _i64,          # host seq_lens, batch, max, total
            _ptr, _i64,                      # plan buffer, bytes
        ],
    ),
    "nie_paged_decode_append_planned": (
        _i32,
        [
            _i32, _ptr, _i64, _i64,          # dtype, q, q strides
            _ptr, _i64, _ptr, _i64,          # new K rows, stride, new V rows, stride
            _ptr, _ptr, _i64,                # RoPE cos / sin tables, rows
            _ptr, _ptr,                      # caches
            _i64, _i64, _i64, _i64,          # layers, layer, blocks, block_size
            _i64, _i64, _i64,                # q_heads, kv_heads, head_dim
            _ptr, _i64,                      # block tables, stride
            _ptr, _i64, _i64, _i64,          # seq_lens, batch, max bound, total bound
            _f32,                            # scale
            _ptr, _i64, _i64,                # out, strides
            _ptr, _i64,                      # workspace, bytes
            _ptr, _ptr,                      # device plan, stream
        ],
    ),
    "nie_paged_decode_noalloc_max_bytes": (_i64, []),
    "nie_paged_decode_append_noalloc": (
        _i32,
        [
            _i32, _ptr, _i64, _i64,          # dtype, q, q strides
            _ptr, _i64, _ptr, _i64,          # new K rows, stride, new V rows, stride
            _ptr, _ptr, _i64,                # RoPE cos / sin tables, rows
            _ptr, _ptr,                      # caches
            _i64, _i64, _i64, _i64,          # layers, layer, blocks, block_size
            _i64, _i64, _i64,                # q_heads, kv_heads, head_dim
            _ptr, _i64,                      # block tables, stride
            _ptr, _i64, _i64, _i64,          # seq_lens, batch, max, total
            _f32,                            # scale
            _ptr, _i64, _i64,                # out, strides
            _ptr, _ptr,                      # host seq_lens, stream
        ],
    ),
    "nie_varlen_prefill_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr]),
    "nie_varlen_prefill": (
        _i32,
        [
            _i32, _ptr, _i64, _i64,          # dtype, q, q strides
            _ptr, _ptr, _i64, _i64,          # cu_seqlens, context_lens, num_seqs, total_q
            _i64, _i64,                      # max_q, max_seq
            _ptr, _ptr,                      # caches
            _i64, _i64, _i64, _i64,          # layers, layer, blocks, block_size
            _i64, _i64, _i64,                # q_heads, kv_heads, head_dim
            _ptr, _i64,                      # block tables, stride
            _f32,                            # scale
            _ptr, _i64, _i64,                # out, strides
            _ptr, _i64,                      # workspace, bytes
            _ptr, _ptr, _ptr,                # host cu_seqlens, host context_lens, stream
        ],
    ),
}

_lib: ctypes.CDLL | None = None
_lib_lock = threading.Lock()

# Split-partial workspaces of the decode and prefill calls, one per (device,
# stream), grown as needed and reused: calls on one stream are ordered, so
# they can share a buffer; calls on different streams cannot.  Each starts
# zeroed: its first workspace_control_bytes() bytes are the library's
# control region, which must be zero before first use (calls leave it zero).
_decode_workspaces: dict[tuple[int, int], torch.Tensor] = {}
_workspace_lock = threading.Lock()


def _decode_workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    with _workspace_lock:
        ws = _decode_workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            size = max(nbytes, 1 << 20, 0 if ws is None else 2 * ws.numel())
            ws = torch.zeros(size, dtype=torch.uint8, device=device)
            _decode_workspaces[key] = ws
    return ws


def _host_lengths(cu_seqlens_host, context_lens_host, num_seqs: int):
    """Host copies of cu_seqlens / context_lens as C arrays (or (None, None)).

    Given, they let the library plan a prefill launch from the exact work;
    they must hold the same values as the device tensors.
    """
    if cu_seqlens_host is None or context_lens_host is None:
        return None, None
    cu = np.ascontiguousarray(np.asarray(cu_seqlens_host, dtype=np.int64))
    ctx = np.ascontiguousarray(np.asarray(context_lens_host, dtype=np.int32))
    if cu.shape != (num_seqs + 1,) or ctx.shape != (num_seqs,):
        raise ValueError("host cu_seqlens / context_lens must have num_seqs + 1 / num_seqs entries")
    return cu, ctx


def _host_seq_lens(seq_lens_host, batch: int):
    """Host copy of a decode call's lengths as a C int32 array (or None)."""
    if seq_lens_host is None:
        return None
    lens = np.ascontiguousarray(np.asarray(seq_lens_host, dtype=np.int32))
    if lens.shape != (batch,):
        raise ValueError("host seq_lens must have batch entries")
    return lens


def _array_ptr(a) -> int | None:
    return None if a is None else a.ctypes.data


def library_path() -> str:
    """Path of the in-tree built library."""
    override = os.environ.get("NIE_HIP_LIBRARY")
    if override:
        return override
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), LIBRARY_NAME)


def load_library() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is None:
            path = library_path()
            if not os.path.exists(path):
                raise RuntimeError(
                    f"HIP paged-attention library not found at {path}; "
                    "build it with `python -c 'import __graft_entry__ as g; g.build()'`"
                )
            lib = ctypes.CDLL(path)
            for name, (restype, argtypes) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = lib
    return _lib


def version() -> str:
    return load_library().nie_version().decode()


def set_attention_rounding(mode: str) -> None:
    """Where the bf16 attention kernels round the softmax probabilities, for
    every launch made after this call in the process.

    ``"reference"`` (the default): the reference's rounding point, the
    normalised probabilities exp(s - m) / l cast to bf16 before P.V
    (``layers/paged_attention.py:109-114``, ``layers/attention.py:410-411``),
    with two passes over the keys.  ``"fast"``: one pass with an online
    softmax, exp(s - running max) cast to bf16 and the row divided by its sum
    at the end.  Prepared launches size their workspace for the mode of the
    moment they are built.
    """
    if mode not in ROUNDING_MODES:
        raise ValueError(f"attention rounding must be one of {sorted(ROUNDING_MODES)}, not {mode!r}")
    _check(load_library().nie_set_attention_rounding(ROUNDING_MODES[mode]), "nie_set_attention_rounding")


def attention_rounding() -> str:
    """The rounding mode of ``set_attention_rounding``."""
    code = load_library().nie_attention_rounding()
    return next(name for name, value in ROUNDING_MODES.items() if value == code)


#: Paths of a decode call (nie_decode_last_path).
DECODE_PATHS = {0: "none", 1: "one_pass", 2: "passes", 3: "fused", 4: "generic", 5: "one_pass_merged"}


def set_decode_fused(on: bool | int) -> None:
    """Whether reference-rounding bf16 decode calls whose shape allows it run
    as one kernel (each split keeps its scores on chip and the splits exchange
    only their (max, sum) pairs) instead of the scores and P.V passes, and
    whether small one-pass decode calls that split their keys merge the
    splits inside the decode kernel (the last split of each (sequence, KV
    head) merges) instead of a merge launch; the outputs are bit-identical
    either way.  On by default; process-wide.  2: as on, and the one-pass
    merge by the last split in calls of every size."""
    value = int(on) if not isinstance(on, bool) else (1 if on else 0)
    _check(load_library().nie_set_decode_fused(value), "nie_set_decode_fused")


def decode_fused() -> int:
    """The switch's value: 0 off, 1 on (the default), 2 on with every
    one-pass call merged by its last split."""
    return int(load_library().nie_decode_fused())


def set_decode_fused_spin(polls: int) -> None:
    """Polls a split of the one-launch decode makes while waiting for the
    other splits of its sequence before it forms their statistics itself (0:
    give up at once, the path tests use to run that code)."""
    _check(load_library().nie_set_decode_fused_spin(int(polls)), "nie_set_decode_fused_spin")


def workspace_control_bytes() -> int:
    """Bytes at the start of a decode or prefill workspace that hold the control region."""
    return int(load_library().nie_workspace_control_bytes())


def decode_last_path() -> str:
    """Which kernels this thread's last decode call ran ("fused", "passes", ...)."""
    return DECODE_PATHS[load_library().nie_decode_last_path()]


def _check(rc: int, what: str) -> None:
    if rc != 0:
        message = load_library().nie_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {message}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise RuntimeError(f"HIP kernels support float32 and bfloat16, not {dtype}") from None


def _require_gpu(*tensors: torch.Tensor) -> None:
    for tensor in tensors:
        if tensor.device.type != "cuda":
            raise RuntimeError(
                "paged KV operations run on a ROCm GPU through the HIP library; "
                f"got a tensor on {tensor.device}"
            )


# The current stream's raw handle straight from torch's C++ side (0.1 us a
# call against about 2 us for ``torch.cuda.current_stream(device).cuda_stream``,
# which builds a Stream object); the public route where torch lacks it.
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    if _RAW_STREAM is not None:
        return _RAW_STREAM(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def _cache_dims(k_cache: torch.Tensor) -> tuple[int, int, int, int, int]:
    if k_cache.ndim != 5:
        raise ValueError("key_cache and value_cache must be 5D tensors")
    if not k_cache.is_contiguous():
        raise ValueError("KV cache storage must be contiguous")
    return tuple(k_cache.shape)  # type: ignore[return-value]


def _check_cache_pair(k_cache: torch.Tensor, v_cache: torch.Tensor) -> tuple[int, int, int, int, int]:
    _require_gpu(k_cache, v_cache)
    dims = _cache_dims(k_cache)
    if v_cache.shape != k_cache.shape or not v_cache.is_contiguous():
        raise ValueError("key_cache and value_cache must have identical contiguous shapes")
    if v_cache.dtype != k_cache.dtype or v_cache.device != k_cache.device:
        raise ValueError("key_cache and value_cache must share dtype and device")
    return dims


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """``t`` itself if its storage pointer is 16-byte aligned, else an aligned copy."""
    if t.data_ptr() % 16 == 0:
        return t
    return t.clone(memory_format=torch.contiguous_format)


def _rows_view_ok(t: torch.Tensor, kv_heads: int, head_dim: int) -> bool:
    return t.ndim == 3 and t.shape[1:] == (kv_heads, head_dim) and t.stride(2) == 1 and t.stride(1) == head_dim


def kv_append(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    layer_index: int,
    keys: torch.Tensor,
    values: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> None:
    """Write token t of ``keys``/``values`` (T, Hkv, D) to slot ``slot_mapping[t]``."""
    num_layers, num_blocks, block_size, kv_heads, head_dim = _check_cache_pair(k_cache, v_cache)
    _require_gpu(keys, values, slot_mapping)
    if keys.dtype != k_cache.dtype or values.dtype != k_cache.dtype:
        raise ValueError("keys and values must match the cache dtype")
    if slot_mapping.dtype != torch.int64 or slot_mapping.ndim != 1 or not slot_mapping.is_contiguous():
        raise ValueError("slot_mapping must be a contiguous 1D int64 tensor")
    if keys.shape != values.shape or keys.shape[0] != slot_mapping.shape[0]:
        raise ValueError("keys, values and slot_mapping must describe the same tokens")
    if not _rows_view_ok(keys, kv_heads, head_dim):
        keys = keys.contiguous()
    if not _rows_view_ok(values, kv_heads, head_dim):
        values = values.contiguous()
    lib = load_library()
    rc = lib.nie_kv_append(
        dtype_code(k_cache.dtype),
        keys.data_ptr(), keys.stride(0),
        values.data_ptr(), values.stride(0),
        slot_mapping.data_ptr(), slot_mapping.shape[0],
        k_cache.data_ptr(), v_cache.data_ptr(),
        num_layers, layer_index, num_blocks, block_size, kv_heads, head_dim,
        _stream(k_cache.device),
    )
    _check(rc, "nie_kv_append")


def _check_rope_inputs(q, k, v, positions, slot_mapping, cos_table, sin_table, dtype, kv_heads, head_dim):
    _require_gpu(q, k, v, positions, slot_mapping, cos_table, sin_table)
    tokens = positions.shape[0] if positions.ndim == 1 else -1
    for name, t in (("positions", positions), ("slot_mapping", slot_mapping)):
        if t.dtype != torch.int64 or t.ndim != 1 or t.shape[0] != tokens or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous 1D int64 tensor with one entry per token")
    for name, t, heads in (("q", q, None), ("k", k, kv_heads), ("v", v, kv_heads)):
        if t.dtype != dtype or t.ndim != 3 or t.shape[0] != tokens or t.shape[2] != head_dim or t.stride(2) != 1:
            raise ValueError(f"{name} must be (tokens, heads, head_dim) rows in the cache dtype")
        if heads is not None and t.shape[1] != heads:
            raise ValueError(f"{name} must have {heads} heads")
    half = head_dim // 2
    for name, t in (("cos_table", cos_table), ("sin_table", sin_table)):
        if t.dtype != dtype or t.ndim != 2 or t.shape[1] != half or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous (positions, head_dim / 2) tensor in the cache dtype")
    if cos_table.shape != sin_table.shape or cos_table.shape[0] == 0:
        raise ValueError("cos_table and sin_table must have the same non-empty shape")


def rope_kv_append(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    layer_index: int,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    positions: torch.Tensor,
    slot_mapping: torch.Tensor,
    cos_table: torch.Tensor,
    sin_table: torch.Tensor,
) -> None:
    """RoPE of q (in place) and k at ``positions``, then k/v rows to slot ``slot_mapping[t]``.

    ``cos_table``/``sin_table`` row p holds cos/sin of p * inv_freq in the
    cache dtype; every position must have a row (checked on the host when the
    positions are host-visible, clamped on the device otherwise).
    """
    num_layers, num_blocks, block_size, kv_heads, head_dim = _check_cache_pair(k_cache, v_cache)
    _check_rope_inputs(q, k, v, positions, slot_mapping, cos_table, sin_table, k_cache.dtype, kv_heads, head_dim)
    lib = load_library()
    rc = lib.nie_rope_kv_append(
        dtype_code(k_cache.dtype),
        q.data_ptr(), q.stride(0), q.stride(1), q.shape[1],
        k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1),
        positions.data_ptr(), slot_mapping.data_ptr(), positions.shape[0],
        cos_table.data_ptr(), sin_table.data_ptr(), cos_table.shape[0],
        k_cache.data_ptr(), v_cache.data_ptr(),
        num_layers, layer_index, num_blocks, block_size, kv_heads, head_dim,
        _stream(k_cache.device),
    )
    _check(rc, "nie_rope_kv_append")


ARGMAX_PIECE_COLS = 8192


def argmax_rows(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Index of the largest value of each row of a 2D logits tensor (torch.argmax(dim=-1) semantics), int64."""
    _require_gpu(logits)
    if logits.ndim != 2 or logits.shape[1] == 0 or logits.stride(1) != 1:
        raise ValueError("logits must be a 2D tensor with contiguous, non-empty rows")
    rows = logits.shape[0]
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    elif out.dtype != torch.int64 or out.shape != (rows,) or not out.is_contiguous() or out.device != logits.device:
        raise ValueError("out must be a contiguous int64 tensor with one entry per row")
    cols = logits.shape[1]
    stride = logits.stride(0) if rows > 1 else cols
    lib = load_library()
    if cols >= 2 * ARGMAX_PIECE_COLS:
        # long rows (an LM head's logits): one workgroup per piece of a row,
        # then a merge of the pieces' (value, index) pairs
        ws_bytes = lib.nie_argmax_rows_workspace_bytes(rows, cols)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=logits.device)
        rc = lib.nie_argmax_rows_split(dtype_code(logits.dtype), logits.data_ptr(), rows, cols, stride,
                                       out.data_ptr(), ws.data_ptr(), ws_bytes, _stream(logits.device))
        _check(rc, "nie_argmax_rows_split")
        return out
    rc = lib.nie_argmax_rows(dtype_code(logits.dtype), logits.data_ptr(), rows, cols, stride, out.data_ptr(),
                             _stream(logits.device))
    _check(rc, "nie_argmax_rows")
    return out


def _norm_rows(t: torch.Tensor, cols: int) -> torch.Tensor:
    """t as (rows, cols) with unit column stride and 16-byte row strides (a view when possible)."""
    t2 = t.reshape(-1, cols)
    if t2.stride(1) != 1 or (t2.shape[0] > 1 and (t2.stride(0) * t2.element_size()) % 16):
        t2 = t2.contiguous()
    return t2


def rms_norm_supported(x: torch.Tensor) -> bool:
    """Whether nie_rms_norm / nie_silu_mul take x's dtype and row length."""
    if x.dtype not in _DTYPE_CODES or x.ndim == 0:
        return False
    per_vec = 16 // x.element_size()
    return x.shape[-1] % per_vec == 0 and 0 < x.shape[-1] <= 1024 * per_vec


def silu_mul_supported(x: torch.Tensor) -> bool:
    """Whether nie_silu_mul takes x's dtype and row length."""
    return x.dtype in _DTYPE_CODES and x.ndim > 0 and x.shape[-1] % (16 // x.element_size()) == 0


def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float, residual: torch.Tensor | None = None):
    """RMSNorm over the last dimension (``layers/rms_norm.py:25-31`` arithmetic, fp32 inside).

    With ``residual`` returns ``(x + residual, norm(x + residual))``, the sum
    rounded to x's dtype as torch's addition does; otherwise ``norm(x)``.
    """
    _require_gpu(x)
    cols = x.shape[-1]
    if not rms_norm_supported(x):
        raise RuntimeError(f"nie_rms_norm does not take {x.dtype} rows of {cols} elements")
    xs = _aligned(_norm_rows(x, cols))
    rows = xs.shape[0]
    out = torch.empty((rows, cols), dtype=x.dtype, device=x.device)
    w = None
    if weight is not None:
        if weight.shape != (cols,) or weight.device != x.device or weight.dtype != x.dtype:
            raise ValueError("weight must be a (cols,) tensor of x's dtype on the device of x")
        w = _aligned(weight.detach().contiguous())
    rs = sum_out = None
    if residual is not None:
        if residual.shape != x.shape or residual.dtype != x.dtype or residual.device != x.device:
            raise ValueError("residual must match x")
        rs = _aligned(_norm_rows(residual, cols))
        sum_out = torch.empty((rows, cols), dtype=x.dtype, device=x.device)
    rc = load_library().nie_rms_norm(
        dtype_code(x.dtype), xs.data_ptr(), xs.stride(0) if rows > 1 else cols,
        None if rs is None else rs.data_ptr(), 0 if rs is None else (rs.stride(0) if rows > 1 else cols),
        None if sum_out is None else sum_out.data_ptr(), cols,
        None if w is None else w.data_ptr(), out.data_ptr(), cols, rows, cols, float(eps), _stream(x.device),
    )
    _check(rc, "nie_rms_norm")
    if sum_out is None:
        return out.view(x.shape)
    return sum_out.view(x.shape), out.view(x.shape)


def rms_norm_rows_into(x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor, eps: float,
                       out: torch.Tensor, sum_out: torch.Tensor | None, stream: int) -> None:
    """``nie_rms_norm`` over contiguous (rows, cols) tensors the caller made:
    ``out = norm(x [+ residual])`` (and ``sum_out = x + residual``), weight
    (cols,).  No Python-side checks beyond the library's own: for the
    packed-token blocks (``Llama3Decoder.forward_tokens_lean``), whose
    buffers are allocated right before the call."""
    rows, cols = x.shape
    rc = load_library().nie_rms_norm(
        _DTYPE_CODES[x.dtype], x.data_ptr(), cols, None if residual is None else residual.data_ptr(), cols,
        None if sum_out is None else sum_out.data_ptr(), cols, weight.data_ptr(), out.data_ptr(), cols, rows, cols,
        eps, stream,
    )
    if rc:
        _check(rc, "nie_rms_norm")


def silu_mul_rows(gate_up: torch.Tensor, inner: int, stream: int) -> torch.Tensor:
    """``silu(gate) * up`` of a contiguous (rows, 2 * inner) ``[gate | up]``
    projection the caller made (``Llama3Decoder.forward_tokens_lean``); the
    halves are read with their row stride.  No Python-side checks beyond
    the library's own."""
    rows = gate_up.shape[0]
    out = torch.empty((rows, inner), dtype=gate_up.dtype, device=gate_up.device)
    base = gate_up.data_ptr()
    rc = load_library().nie_silu_mul(_DTYPE_CODES[gate_up.dtype], base, 2 * inner,
                                     base + inner * gate_up.element_size(), 2 * inner, out.data_ptr(), inner, rows,
                                     inner, stream)
    if rc:
        _check(rc, "nie_silu_mul")
    return out


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up with torch's roundings (``layers/mlp.py:18-22``).

    gate and up may be row-strided views (the halves of a fused gate/up
    projection's output); the result is contiguous.
    """
    _require_gpu(gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype or gate.device != up.device:
        raise ValueError("gate and up must have the same shape, dtype and device")
    if not silu_mul_supported(gate):
        raise RuntimeError(f"nie_silu_mul does not take {gate.dtype} tensors of shape {tuple(gate.shape)}")
    cols = gate.shape[-1]
    g = _aligned(_norm_rows(gate, cols))
    u = _aligned(_norm_rows(up, cols))
    rows = g.shape[0]
    out = torch.empty((rows, cols), dtype=gate.dtype, device=gate.device)
    rc = load_library().nie_silu_mul(dtype_code(g.dtype), g.data_ptr(), g.stride(0) if rows > 1 else cols,
                                     u.data_ptr(), u.stride(0) if rows > 1 else cols, out.data_ptr(), cols, rows,
                                     cols, _stream(g.device))
    _check(rc, "nie_silu_mul")
    return out.view(gate.shape)


LINEAR_MAX_ROWS = 16
#: In-feature sizes nie_linear_rows is built for; the SiLU epilogue only for the first two.
LINEAR_K_BUILT = (2048, 4096, 8192)
LINEAR_K_BUILT_SILU = (2048, 4096)
LINEAR_PLAIN = 0
LINEAR_SILU_MUL = 1


def linear_rows_supported(x: torch.Tensor, weight: torch.Tensor, silu_mul: bool = False) -> bool:
    """Whether nie_linear_rows takes ``F.linear(x, weight)`` (with the SwiGLU
    epilogue when ``silu_mul``): bf16 on the GPU, at most 16 rows, an
    in-feature size the library is built for, out-features a multiple of 16."""
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or weight.ndim != 2 or x.ndim == 0:
        return False
    if not x.is_cuda or weight.device != x.device:
        return False
    n, k = weight.shape
    return x.shape[-1] == k and linear_rows_shape_built(x.numel() // max(k, 1), n, k, silu_mul)


def linear_rows_shape_built(rows: int, n: int, k: int, silu_mul: bool = False) -> bool:
    """The shapes nie_linear_rows is built for (its NIE_EUNSUPPORTED check on
    the host): 1..16 rows, n a positive multiple of 16 (of 32 for a
    ``[gate; up]`` weight), k in 2048 / 4096, or 8192 without the SiLU epilogue."""
    built = LINEAR_K_BUILT_SILU if silu_mul else LINEAR_K_BUILT
    return 0 < rows <= LINEAR_MAX_ROWS and k in built and n > 0 and n % (32 if silu_mul else 16) == 0


def linear_rows(x: torch.Tensor, weight: torch.Tensor, silu_mul: bool = False) -> torch.Tensor:
    """``F.linear(x, weight)`` (no bias) for a decode step's few rows, on nie_linear_rows.

    With ``silu_mul`` the weight is a SwiGLU block's ``[gate; up]`` rows and the
    result is ``silu(gate) * up`` (``layers/mlp.py:18-22``), half as wide.
    """
    _require_gpu(x, weight)
    if not linear_rows_supported(x, weight, silu_mul):
        raise RuntimeError(f"nie_linear_rows does not take x {tuple(x.shape)} {x.dtype} with weight "
                           f"{tuple(weight.shape)} {weight.dtype}" + (" and the SiLU epilogue" if silu_mul else ""))
    n, k = weight.shape
    n_out = n // 2 if silu_mul else n
    xs = _aligned(_norm_rows(x, k))
    w = _aligned(weight.detach() if weight.is_contiguous() else weight.detach().contiguous())
    rows = xs.shape[0]
    out = torch.empty((rows, n_out), dtype=x.dtype, device=x.device)
    rc = load_library().nie_linear_rows(
        dtype_code(x.dtype), xs.data_ptr(), xs.stride(0) if rows > 1 else k, rows, w.data_ptr(), n_out, k,
        LINEAR_SILU_MUL if silu_mul else LINEAR_PLAIN, out.data_ptr(), n_out, _stream(x.device),
    )
    _check(rc, "nie_linear_rows")
    return out.view(*x.shape[:-1], n_out)


RMS_NORM_LINEAR_K = 2048


def rms_norm_linear_rows(
    x: torch.Tensor,
    residual: torch.Tensor | None,
    norm_weight: torch.Tensor,
    eps: float,
    weight: torch.Tensor,
    silu_mul: bool = False,
    want_sum: bool = True,
) -> tuple[torch.Tensor | None, torch.Tensor]:
    """``RmsNorm(x + residual)`` then ``F.linear(., weight)`` in one launch (nie_rms_norm_linear_rows).

    Returns ``(x + residual, y)`` (the sum is None without a residual or with
    ``want_sum=False``); ``silu_mul`` as for :func:`linear_rows`.  The norm's
    arithmetic is ``rms_norm``'s (``layers/rms_norm.py:25-31``).
    """
    _require_gpu(x, weight, norm_weight)
    if not linear_rows_supported(x, weight, silu_mul) or weight.shape[1] != RMS_NORM_LINEAR_K:
        raise RuntimeError(f"nie_rms_norm_linear_rows does not take x {tuple(x.shape)} {x.dtype} with weight "
                           f"{tuple(weight.shape)} {weight.dtype}")
    n, k = weight.shape
    if norm_weight.shape != (k,) or norm_weight.dtype != x.dtype or norm_weight.device != x.device:
        raise ValueError("norm_weight must be a (k,) tensor of x's dtype on the device of x")
    if residual is not None and (residual.shape != x.shape or residual.dtype != x.dtype
                                 or residual.device != x.device):
        raise ValueError("residual must match x")
    n_out = n // 2 if silu_mul else n
    xs = _aligned(_norm_rows(x, k))
    rows = xs.shape[0]
    rs = None if residual is None else _aligned(_norm_rows(residual, k))
    nw = _aligned(norm_weight.detach().contiguous())
    w = _aligned(weight.detach() if weight.is_contiguous() else weight.detach().contiguous())
    out = torch.empty((rows, n_out), dtype=x.dtype, device=x.device)
    sum_out = torch.empty((rows, k), dtype=x.dtype, device=x.device) if (want_sum and rs is not None) else None
    rc = load_library().nie_rms_norm_linear_rows(
        dtype_code(x.dtype), xs.data_ptr(), xs.stride(0) if rows > 1 else k,
        None if rs is None else rs.data_ptr(), 0 if rs is None else (rs.stride(0) if rows > 1 else k),
        None if sum_out is None else sum_out.data_ptr(), k, nw.data_ptr(), float(eps), rows, w.data_ptr(), n_out, k,
        LINEAR_SILU_MUL if silu_mul else LINEAR_PLAIN, out.data_ptr(), n_out, _stream(x.device),
    )
    _check(rc, "nie_rms_norm_linear_rows")
    return (None if sum_out is None else sum_out.view(x.shape)), out.view(*x.shape[:-1], n_out)


def kv_gather(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    layer_index: int,
    block_table: torch.Tensor,
    token_count: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Contiguous (token_count, Hkv, D) copies of logical positions 0..token_count-1."""
    num_layers, num_blocks, block_size, kv_heads, head_dim = _check_cache_pair(k_cache, v_cache)
    _require_gpu(block_table)
    if block_table.dtype != torch.int32 or block_table.ndim != 1 or not block_table.is_contiguous():
        raise ValueError("block_table must be a contiguous 1D int32 tensor")
    k_out = torch.empty((token_count, kv_heads, head_dim), dtype=k_cache.dtype, device=k_cache.device)
    v_out = torch.empty_like(k_out)
    rc = load_library().nie_kv_gather(
        dtype_code(k_cache.dtype),
        k_cache.data_ptr(), v_cache.data_ptr(),
        num_layers, layer_index, num_blocks, block_size, kv_heads, head_dim,
        block_table.data_ptr(), block_table.shape[0], token_count,
        k_out.data_ptr(), v_out.data_ptr(),
        _stream(k_cache.device),
    )
    _check(rc, "nie_kv_gather")
    return k_out, v_out


def kv_copy_blocks(
    src_k: torch.Tensor,
    src_v: torch.Tensor,
    src_blocks: torch.Tensor | None,
    dst_k: torch.Tensor,
    dst_v: torch.Tensor,
    dst_blocks: torch.Tensor | None,
    count: int,
) -> None:
    """Copy ``count`` whole blocks (all layers, K and V).

    A side whose block list is ``None`` is a packed staging tensor of shape
    (L, count, BS, Hkv, D); otherwise it is a pool indexed by the list.
    """
    for t in (src_k, src_v, dst_k, dst_v):
        if t.ndim != 5 or not t.is_contiguous():
            raise ValueError("block copies need contiguous 5D K/V tensors")
    # the kernel indexes V with K's geometry, and a packed side with `count`
    # as its per-layer block count
    if src_v.shape != src_k.shape or dst_v.shape != dst_k.shape:
        raise ValueError("V tensors must have the shape of their K tensors")
    if src_k.shape[0] != dst_k.shape[0] or src_k.shape[2:] != dst_k.shape[2:]:
        raise ValueError("source and destination layouts differ")
    if src_k.dtype != dst_k.dtype or src_v.dtype != src_k.dtype or dst_v.dtype != dst_k.dtype:
        raise ValueError("source and destination dtypes differ")
    if count < 0:
        raise ValueError("count must be non-negative")
    for side, blocks, pool in (("source", src_blocks, src_k), ("destination", dst_blocks, dst_k)):
        if blocks is None:
            if pool.shape[1] != count:
                raise ValueError(f"a packed {side} must hold exactly `count` blocks per layer")
        elif blocks.dtype != torch.int32 or blocks.ndim != 1 or blocks.shape[0] < count:
            raise ValueError("block lists must be 1D int32 tensors with `count` entries")
    _require_gpu(src_k, src_v, dst_k, dst_v, *(b for b in (src_blocks, dst_blocks) if b is not None))
    num_layers, _, block_size, kv_heads, head_dim = src_k.shape
    rc = load_library().nie_kv_copy_blocks(
        dtype_code(src_k.dtype),
        src_k.data_ptr(), src_v.data_ptr(), src_k.shape[1],
        None if src_blocks is None else src_blocks.data_ptr(),
        dst_k.data_ptr(), dst_v.data_ptr(), dst_k.shape[1],
        None if dst_blocks is None else dst_blocks.data_ptr(),
        count, num_layers, block_size, kv_heads, head_dim,
        _stream(src_k.device),
    )
    _check(rc, "nie_kv_copy_blocks")


def _check_attention_shapes(q_heads: int, kv_heads: int, head_dim: int) -> None:
    if not 0 < head_dim <= GENERIC_MAX_HEAD_DIM:
        raise RuntimeError(f"HIP attention supports head_dim 1 to {GENERIC_MAX_HEAD_DIM}, not {head_dim}")
    if q_heads <= 0 or kv_heads <= 0 or q_heads % kv_heads != 0:
        raise RuntimeError(f"q_heads must be a positive multiple of kv_heads; got {q_heads}/{kv_heads}")


def paged_decode(
    query: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    layer_index: int,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    max_seq_len: int,
    total_seq_len: int,
    scale: float,
    out: torch.Tensor | None = None,
    seq_lens_host=None,
    new_kv: tuple[torch.Tensor, torch.Tensor] | None = None,
    rope_tables: tuple[torch.Tensor, torch.Tensor] | None = None,
) -> torch.Tensor:
    """Decode attention of query (B, Hq, D) over each sequence's first seq_lens[b] tokens.

    ``block_tables`` (B, W) int32 and ``seq_lens`` (B,) int32 are device
    tensors; ``max_seq_len`` and ``total_seq_len`` are their host-side max
    and sum (they size the launch and must be exact).  The optional
    ``seq_lens_host`` (ints equal to ``seq_lens``) lets the launch be planned
    from the exact lengths.

    ``new_kv=(keys, values)``, each (B, Hkv, D): the same launch first
    writes row b at position seq_lens[b] - 1 (the slot its block table
    gives), as the decode step of ``GroupedQueryAttention.forward`` writes
    the new token before attending (reference ``layers/attention.py:246-269``).
    ``rope_tables=(cos, sin)``, each (rows, D/2) in the storage dtype (with
    ``new_kv`` only): q and the new K rows are first rotated at that position
    as ``rope_kv_append`` rotates them; q itself is not modified.
    """
    num_layers, num_blocks, block_size, kv_heads, head_dim = _check_cache_pair(k_cache, v_cache)
    _require_gpu(query, block_tables, seq_lens)
    if query.ndim != 3 or query.shape[2] != head_dim or query.stride(2) != 1:
        raise ValueError("query must be (batch, q_heads, head_dim) with unit stride on head_dim")
    if query.dtype != k_cache.dtype:
        raise ValueError("query and K/V caches must have the same dtype")
    query = _aligned(query)
    batch, q_heads, _ = query.shape
    _check_attention_shapes(q_heads, kv_heads, head_dim)
    if block_tables.dtype != torch.int32 or block_tables.ndim != 2 or block_tables.shape[0] != batch:
        raise ValueError("block_tables must be an int32 (batch, max_blocks) tensor")
    if not block_tables.is_contiguous():
        block_tables = block_tables.contiguous()
    if seq_lens.dtype != torch.int32 or seq_lens.shape != (batch,) or not seq_lens.is_contiguous():
        raise ValueError("seq_lens must be a contiguous int32 (batch,) tensor")
    if out is None:
        out = torch.empty((batch, q_heads, head_dim), dtype=query.dtype, device=query.device)
    if batch == 0:
        return out
    host_lens = _host_seq_lens(seq_lens_host, batch)
    lib = load_library()
    ws_bytes = lib.nie_paged_decode_workspace_bytes(
        dtype_code(query.dtype), batch, q_heads, kv_heads, head_dim, block_size, max_seq_len, total_seq_len,
        _array_ptr(host_lens),
    )
    stream = _stream(query.device)
    workspace = _decode_workspace(query.device, stream, ws_bytes)
    if rope_tables is not None and new_kv is None:
        raise ValueError("rope_tables applies to the fused append (new_kv)")
    if new_kv is not None:
        align = _row_align(q_heads, kv_heads, head_dim)
        keys, values = _check_new_rows(new_kv, batch, kv_heads, head_dim, query.dtype, query.device, align)
        cos, sin, rows = _check_rope_tables(rope_tables, head_dim, query.dtype, query.device, align)
        rc = lib.nie_paged_decode_append(
            dtype_code(query.dtype),
            query.data_ptr(), query.stride(0), query.stride(1),
            keys.data_ptr(), keys.stride(0), values.data_ptr(), values.stride(0),
            cos, sin, rows,
            k_cache.data_ptr(), v_cache.data_ptr(),
            num_layers, layer_index, num_blocks, block_size,
            q_heads, kv_heads, head_dim,
            block_tables.data_ptr(), block_tables.shape[1],
            seq_lens.data_ptr(), batch, max_seq_len, total_seq_len,
            float(scale),
            out.data_ptr(), out.stride(0), out.stride(1),
            workspace.data_ptr(), workspace.numel(),
            _array_ptr(host_lens),
            stream,
        )
        _check(rc, "nie_paged_decode_append")
        return out
    rc = lib.nie_paged_decode(
        dtype_code(query.dtype),
        query.data_ptr(), query.stride(0), query.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(),
        num_layers, layer_index, num_blocks, block_size,
        q_heads, kv_heads, head_dim,
        block_tables.data_ptr(), block_tables.shape[1],
        seq_lens.data_ptr(), batch, max_seq_len, total_seq_len,
        float(scale),
        out.data_ptr(), out.stride(0), out.stride(1),
        workspace.data_ptr(), workspace.numel(),
        _array_ptr(host_lens),
        stream,
    )
    _check(rc, "nie_paged_decode")
    return out


def _check_rope_tables(rope_tables, head_dim: int, dtype, device, align: int = 16):
    """(cos pointer, sin pointer, rows) of optional RoPE tables, (rows, head_dim/2) each; (None, None, 0) without."""
    if rope_tables is None:
        return None, None, 0
    if head_dim % 2:
        raise ValueError("RoPE needs an even head_dim")
    cos, sin = rope_tables
    for t in (cos, sin):
        if (t.dtype != dtype or t.device != device or t.ndim != 2 or t.shape[1] != head_dim // 2
                or not t.is_contiguous() or t.data_ptr() % align or t.shape[0] == 0):
            raise ValueError("RoPE tables must be contiguous, aligned (rows, head_dim / 2) tensors of the query dtype")
    if cos.shape != sin.shape:
        raise ValueError("RoPE cos and sin tables must have the same shape")
    return cos.data_ptr(), sin.data_ptr(), cos.shape[0]


def _check_new_rows(new_kv, batch: int, kv_heads: int, head_dim: int, dtype, device, align: int = 16):
    """The (keys, values) rows of a fused decode step: (batch, kv_heads, head_dim), rows aligned to ``align`` bytes."""
    keys, values = new_kv
    for t in (keys, values):
        if (t.dtype != dtype or t.device != device or t.shape != (batch, kv_heads, head_dim) or t.stride(2) != 1
                or t.stride(1) != head_dim or t.data_ptr() % align or (t.stride(0) * t.element_size()) % align):
            raise ValueError("new keys/values must be aligned (batch, kv_heads, head_dim) rows matching the query")
    return keys, values


def varlen_prefill(
    query: torch.Tensor,
    cu_seqlens: torch.Tensor,
    context_lens: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    layer_index: int,
    block_tables: torch.Tensor,
    max_query_len: int,
    max_seq_len: int,
    scale: float,
    out: torch.Tensor | None = None,
    cu_seqlens_host=None,
    context_lens_host=None,
) -> torch.Tensor:
    """Causal varlen attention of packed query rows (ΣT, Hq, D) over the paged cache.

    Sequence r owns rows cu_seqlens[r]..cu_seqlens[r+1]-1 at absolute
    positions context_lens[r] + i.  ``max_query_len`` and ``max_seq_len``
    (max of context + query) are exact host-side values.  The optional
    ``cu_seqlens_host`` / ``context_lens_host`` (sequences of ints equal to
    the device tensors) let the launch be planned from the exact work.
    """
    num_layers, num_blocks, block_size, kv_heads, head_dim = _check_cache_pair(k_cache, v_cache)
    _require_gpu(query, cu_seqlens, context_lens, block_tables)
    if query.ndim != 3 or query.shape[2] != head_dim or query.stride(2) != 1:
        raise ValueError("query must be (tokens, q_heads, head_dim) with unit stride on head_dim")
    if query.dtype != k_cache.dtype:
        raise ValueError("query and K/V caches must have the same dtype")
    query = _aligned(query)
    total_tokens, q_heads, _ = query.shape
    _check_attention_shapes(q_heads, kv_heads, head_dim)
    num_seqs = context_lens.shape[0]
    if cu_seqlens.dtype != torch.int64 or cu_seqlens.shape != (num_seqs + 1,) or not cu_seqlens.is_contiguous():
        raise ValueError("cu_seqlens must be a contiguous int64 (num_seqs + 1,) tensor")
    if context_lens.dtype != torch.int32 or not context_lens.is_contiguous():
        raise ValueError("context_lens must be a contiguous int32 tensor")
    if block_tables.dtype != torch.int32 or block_tables.ndim != 2 or block_tables.shape[0] != num_seqs:
        raise ValueError("block_tables must be an int32 (num_seqs, max_blocks) tensor")
    if not block_tables.is_contiguous():
        block_tables = block_tables.contiguous()
    if out is None:
        out = torch.empty((total_tokens, q_heads, head_dim), dtype=query.dtype, device=query.device)
    if total_tokens == 0 or num_seqs == 0:
        return out
    host_cu, host_ctx = _host_lengths(cu_seqlens_host, context_lens_host, num_seqs)
    lib = load_library()
    ws_bytes = lib.nie_varlen_prefill_workspace_bytes(
        num_seqs, total_tokens, max_query_len, max_seq_len, q_heads, kv_heads, head_dim,
        _array_ptr(host_cu), _array_ptr(host_ctx),
    )
    stream = _stream(query.device)
    workspace = _decode_workspace(query.device, stream, ws_bytes) if ws_bytes > 0 else None
    rc = lib.nie_varlen_prefill(
        dtype_code(query.dtype),
        query.data_ptr(), query.stride(0), query.stride(1),
        cu_seqlens.data_ptr(), context_lens.data_ptr(), num_seqs, total_tokens,
        max_query_len, max_seq_len,
        k_cache.data_ptr(), v_cache.data_ptr(),
        num_layers, layer_index, num_blocks, block_size,
        q_heads, kv_heads, head_dim,
        block_tables.data_ptr(), block_tables.shape[1],
        float(scale),
        out.data_ptr(), out.stride(0), out.stride(1),
        None if workspace is None else workspace.data_ptr(), 0 if workspace is None else workspace.numel(),
        _array_ptr(host_cu), _array_ptr(host_ctx),
        stream,
    )
    _check(rc, "nie_varlen_prefill")
    return out


# ---------------------------------------------------------------------------
# Prepared launches: a forward pass runs the same append / decode / prefill
# launch once per layer with only the layer index and the per-layer q, k, v
# and output tensors changing.  These objects check and resolve everything
# else (cache and metadata pointers, launch plan, workspace, stream) once, so
# a layer's launch costs one C call.  They launch on the stream that was
# current when they were built.
# ---------------------------------------------------------------------------
class PreparedAppend:
    """``kv_append`` for one slot mapping, any layer."""

    __slots__ = ("_fn", "_args_cache", "_tokens", "_dtype", "_row_shape", "_device", "_stream", "_slots")

    def __init__(self, k_cache: torch.Tensor, v_cache: torch.Tensor, slot_mapping: torch.Tensor):
        num_layers, num_blocks, block_size, kv_heads, head_dim = _check_cache_pair(k_cache, v_cache)
        _require_gpu(slot_mapping)
        if slot_mapping.dtype != torch.int64 or slot_mapping.ndim != 1 or not slot_mapping.is_contiguous():
            raise ValueError("slot_mapping must be a contiguous 1D int64 tensor")
        self._fn = load_library().nie_kv_append
        self._dtype = k_cache.dtype
        self._device = k_cache.device
        self._row_shape = (kv_heads, head_dim)
        self._tokens = slot_mapping.shape[0]
        self._slots = slot_mapping  # keeps the mapping alive
        self._stream = _stream(k_cache.device)
        self._args_cache = (slot_mapping.data_ptr(), self._tokens, k_cache.data_ptr(), v_cache.data_ptr(),
                            num_layers, num_blocks, block_size, kv_heads, head_dim)

    def __call__(self, keys: torch.Tensor, values: torch.Tensor, layer_index: int) -> None:
        kv_heads, head_dim = self._row_shape
        for t in (keys, values):
            if (t.dtype != self._dtype or t.device != self._device or t.ndim != 3 or t.shape[0] != self._tokens
                    or t.shape[1:] != self._row_shape or t.stride(2) != 1 or t.stride(1) != head_dim):
                raise ValueError("keys/values must be (tokens, kv_heads, head_dim) rows matching the cache")
        slots, tokens, kptr, vptr, num_layers, num_blocks, block_size, _, _ = self._args_cache
        rc = self._fn(_DTYPE_CODES[self._dtype], keys.data_ptr(), keys.stride(0), values.data_ptr(), values.stride(0),
                      slots, tokens, kptr, vptr, num_layers, layer_index, num_blocks, block_size, kv_heads, head_dim,
                      self._stream)
        if rc:
            _check(rc, "nie_kv_append")


class PreparedRopeAppend:
    """``rope_kv_append`` for one batch (positions, slots, sin/cos table), any layer."""

    __slots__ = ("_fn", "_args", "_tokens", "_dtype", "_device", "_kv", "_keep")

    def __init__(self, k_cache: torch.Tensor, v_cache: torch.Tensor, positions: torch.Tensor,
                 slot_mapping: torch.Tensor, cos_table: torch.Tensor, sin_table: torch.Tensor):
        num_layers, num_blocks, block_size, kv_heads, head_dim = _check_cache_pair(k_cache, v_cache)
        tokens = positions.shape[0] if positions.ndim == 1 else 0
        empty = torch.empty((tokens, kv_heads, head_dim), dtype=k_cache.dtype, device=k_cache.device)
        _check_rope_inputs(empty, empty, empty, positions, slot_mapping, cos_table, sin_table, k_cache.dtype,
                           kv_heads, head_dim)
        self._fn = load_library().nie_rope_kv_append
        self._dtype = k_cache.dtype
        self._device = k_cache.device
        self._tokens = tokens
        self._kv = (kv_heads, head_dim)
        self._keep = (positions, slot_mapping, cos_table, sin_table)
        self._args = (positions.data_ptr(), slot_mapping.data_ptr(), tokens, cos_table.data_ptr(),
                      sin_table.data_ptr(), cos_table.shape[0], k_cache.data_ptr(), v_cache.data_ptr(), num_layers,
                      num_blocks, block_size, kv_heads, head_dim, _stream(k_cache.device))

    def __call__(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer_index: int) -> None:
        kv_heads, head_dim = self._kv
        for t, heads in ((q, None), (k, kv_heads), (v, kv_heads)):
            if (t.dtype != self._dtype or t.device != self._device or t.ndim != 3 or t.shape[0] != self._tokens
                    or t.shape[2] != head_dim or t.stride(2) != 1 or (heads is not None and t.shape[1] != heads)):
                raise ValueError("q/k/v must be (tokens, heads, head_dim) rows matching the batch and the cache")
        (pos, slots, tokens, cos, sin, rows, kptr, vptr, num_layers, num_blocks, block_size, _, _,
         stream) = self._args
        rc = self._fn(_DTYPE_CODES[self._dtype], q.data_ptr(), q.stride(0), q.stride(1), q.shape[1], k.data_ptr(),
                      k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), pos, slots, tokens, cos, sin,
                      rows, kptr, vptr, num_layers, layer_index, num_blocks, block_size, kv_heads, head_dim, stream)
        if rc:
            _check(rc, "nie_rope_kv_append")


def decode_plan_bytes() -> int:
    """Bytes of a decode plan (``write_decode_plan``, ``PreparedDecode(device_plan=...)``)."""
    return int(load_library().nie_paged_decode_plan_bytes())


def write_decode_plan(plan_ptr: int, plan_bytes: int, dtype: torch.dtype, q_heads: int, kv_heads: int,
                      head_dim: int, block_size: int, seq_lens_host: np.ndarray, max_seq_len: int,
                      total_seq_len: int) -> None:
    """Writes at host address ``plan_ptr`` the work items a decode launch
    plans from the host lengths ``seq_lens_host`` (contiguous int32), for a
    device copy that a ``device_plan`` launch reads."""
    if seq_lens_host.dtype != np.int32 or not seq_lens_host.flags.c_contiguous:
        raise ValueError("seq_lens_host must be a contiguous int32 array")
    rc = load_library().nie_paged_decode_plan(dtype_code(dtype), q_heads, kv_heads, head_dim, block_size,
                                              seq_lens_host.ctypes.data, seq_lens_host.shape[0], max_seq_len,
                                              total_seq_len, plan_ptr, plan_bytes)
    if rc:
        _check(rc, "nie_paged_decode_plan")


_plan_probe = threading.local()


def decode_plan_fits(dtype: torch.dtype, q_heads: int, kv_heads: int, head_dim: int, block_size: int,
                     seq_lens_host: list[int]) -> bool:
    """Whether the decode plan of these host lengths fits a work-item table
    (``write_decode_plan`` writes a count of 0 otherwise, and a device-planned
    launch then plans from its bounds)."""
    buf = getattr(_plan_probe, "buf", None)
    if buf is None:
        buf = _plan_probe.buf = np.zeros(-(-decode_plan_bytes() // 4), dtype=np.int32)
    lens = np.ascontiguousarray(seq_lens_host, dtype=np.int32)
    write_decode_plan(buf.ctypes.data, buf.nbytes, dtype, q_heads, kv_heads, head_dim, block_size, lens,
                      int(lens.max()), int(lens.sum()))
    return int(buf[0]) > 0


class PreparedDecode:
    """``paged_decode`` for one batch of sequences (tables, lengths), any layer.

    ``device_plan``: a device buffer of ``decode_plan_bytes()`` that holds, when
    the launch runs, the plan ``write_decode_plan`` wrote for the lengths of
    that moment (or zeros: planned on the device); ``max_seq_len`` and
    ``total_seq_len`` are then bounds.  For launches captured once and
    replayed (``append_decode`` only); the result equals the launch prepared
    with those host lengths.
    """

    __slots__ = ("_fn", "_fn_append", "_pre", "_mid", "_post", "_shape", "_dtype", "_device", "_keep", "_kv_shape",
                 "_align", "_plan")

    def __init__(self, k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                 seq_lens: torch.Tensor, max_seq_len: int, total_seq_len: int, q_heads: int, scale: float,
                 seq_lens_host=None, device_plan: torch.Tensor | None = None):
        num_layers, num_blocks, block_size, kv_heads, head_dim = _check_cache_pair(k_cache, v_cache)
        _require_gpu(block_tables, seq_lens)
        _check_attention_shapes(q_heads, kv_heads, head_dim)
        batch = seq_lens.shape[0] if seq_lens.ndim == 1 else -1
        if seq_lens.dtype != torch.int32 or batch <= 0 or not seq_lens.is_contiguous():
            raise ValueError("seq_lens must be a contiguous int32 (batch,) tensor")
        if (block_tables.dtype != torch.int32 or block_tables.ndim != 2 or block_tables.shape[0] != batch
                or not block_tables.is_contiguous()):
            raise ValueError("block_tables must be a contiguous int32 (batch, max_blocks) tensor")
        host_lens = _host_seq_lens(seq_lens_host, batch)
        lib = load_library()
        self._plan = None
        if device_plan is not None:
            if host_lens is not None:
                raise ValueError("a device-planned decode takes no host lengths")
            if (device_plan.device != k_cache.device or device_plan.numel() * device_plan.element_size()
                    < decode_plan_bytes() or device_plan.data_ptr() % 4):
                raise ValueError("device_plan must be a 4-byte aligned buffer of decode_plan_bytes() on the cache's device")
            self._plan = device_plan.data_ptr()
        code = dtype_code(k_cache.dtype)
        ws_bytes = lib.nie_paged_decode_workspace_bytes(code, batch, q_heads, kv_heads, head_dim, block_size,
                                                        max_seq_len, total_seq_len, _array_ptr(host_lens))
        stream = _stream(k_cache.device)
        workspace = _decode_workspace(k_cache.device, stream, ws_bytes)
        self._fn = lib.nie_paged_decode
        self._fn_append = lib.nie_paged_decode_append if self._plan is None else lib.nie_paged_decode_append_planned
        self._dtype = k_cache.dtype
        self._device = k_cache.device
        self._shape = (batch, q_heads, head_dim)
        self._kv_shape = (batch, kv_heads, head_dim)
        self._align = _row_align(q_heads, kv_heads, head_dim)
        self._keep = (block_tables, seq_lens, workspace, host_lens, device_plan)
        self._pre = (code,)
        self._mid = (k_cache.data_ptr(), v_cache.data_ptr(), num_layers)
        self._post = (num_blocks, block_size, q_heads, kv_heads, head_dim, block_tables.data_ptr(),
                      block_tables.shape[1], seq_lens.data_ptr(), batch, max_seq_len, total_seq_len, float(scale),
                      (workspace.data_ptr(), workspace.numel(), _array_ptr(host_lens), stream))

    def __call__(self, query: torch.Tensor, layer_index: int, out: torch.Tensor) -> torch.Tensor:
        if self._plan is not None:
            raise RuntimeError("a device-planned decode runs through append_decode")
        for t in (query, out):
            if (t.shape != self._shape or t.dtype != self._dtype or t.device != self._device or t.stride(2) != 1
                    or t.data_ptr() % self._align):
                raise ValueError("query/out must be aligned (batch, q_heads, head_dim) tensors matching the batch")
        kptr, vptr, num_layers = self._mid
        (num_blocks, block_size, q_heads, kv_heads, head_dim, tables, tstride, lens, batch, max_len, total_len,
         scale, (ws, ws_bytes, hlens, stream)) = self._post
        rc = self._fn(self._pre[0], query.data_ptr(), query.stride(0), query.stride(1), kptr, vptr, num_layers,
                      layer_index, num_blocks, block_size, q_heads, kv_heads, head_dim, tables, tstride, lens, batch,
                      max_len, total_len, scale, out.data_ptr(), out.stride(0), out.stride(1), ws, ws_bytes, hlens,
                      stream)
        if rc:
            _check(rc, "nie_paged_decode")
        return out

    def append_decode(self, query: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, layer_index: int,
                      out: torch.Tensor, rope_tables: tuple[torch.Tensor, torch.Tensor] | None = None) -> torch.Tensor:
        """Writes keys/values row b at position seq_lens[b] - 1, then decodes, in one launch.

        With ``rope_tables=(cos, sin)`` q and the new keys are rotated at that
        position first (``rope_kv_append``'s arithmetic; q is not modified).
        """
        for t in (query, out):
            if (t.shape != self._shape or t.dtype != self._dtype or t.device != self._device or t.stride(2) != 1
                    or t.data_ptr() % self._align):
                raise ValueError("query/out must be aligned (batch, q_heads, head_dim) tensors matching the batch")
        _check_new_rows((keys, values), *self._kv_shape, self._dtype, self._device, self._align)
        cos, sin, rows = _check_rope_tables(rope_tables, self._kv_shape[2], self._dtype, self._device, self._align)
        kptr, vptr, num_layers = self._mid
        (num_blocks, block_size, q_heads, kv_heads, head_dim, tables, tstride, lens, batch, max_len, total_len,
         scale, (ws, ws_bytes, hlens, stream)) = self._post
        rc = self._fn_append(self._pre[0], query.data_ptr(), query.stride(0), query.stride(1), keys.data_ptr(),
                             keys.stride(0), values.data_ptr(), values.stride(0), cos, sin, rows, kptr, vptr,
                             num_layers, layer_index,
                             num_blocks, block_size, q_heads, kv_heads, head_dim, tables, tstride, lens, batch,
                             max_len, total_len, scale, out.data_ptr(), out.stride(0), out.stride(1), ws, ws_bytes,
                             hlens if self._plan is None else self._plan, stream)
        if rc:
            _check(rc, "nie_paged_decode_append")
        return out


class PreparedPrefill:
    """``varlen_prefill`` for one packed ragged batch, any layer."""

    __slots__ = ("_fn", "_args", "_shape", "_dtype", "_device", "_keep", "_align")

    def __init__(self, k_cache: torch.Tensor, v_cache: torch.Tensor, cu_seqlens: torch.Tensor,
                 context_lens: torch.Tensor, block_tables: torch.Tensor, total_tokens: int, max_query_len: int,
                 max_seq_len: int, q_heads: int, scale: float, cu_seqlens_host=None, context_lens_host=None):
        num_layers, num_blocks, block_size, kv_heads, head_dim = _check_cache_pair(k_cache, v_cache)
        _require_gpu(cu_seqlens, context_lens, block_tables)
        _check_attention_shapes(q_heads, kv_heads, head_dim)
        num_seqs = context_lens.shape[0]
        if cu_seqlens.dtype != torch.int64 or cu_seqlens.shape != (num_seqs + 1,) or not cu_seqlens.is_contiguous():
            raise ValueError("cu_seqlens must be a contiguous int64 (num_seqs + 1,) tensor")
        if context_lens.dtype != torch.int32 or not context_lens.is_contiguous():
            raise ValueError("context_lens must be a contiguous int32 tensor")
        if (block_tables.dtype != torch.int32 or block_tables.ndim != 2 or block_tables.shape[0] != num_seqs
                or not block_tables.is_contiguous()):
            raise ValueError("block_tables must be a contiguous int32 (num_seqs, max_blocks) tensor")
        host_cu, host_ctx = _host_lengths(cu_seqlens_host, context_lens_host, num_seqs)
        lib = load_library()
        ws_bytes = lib.nie_varlen_prefill_workspace_bytes(num_seqs, total_tokens, max_query_len, max_seq_len,
                                                          q_heads, kv_heads, head_dim, _array_ptr(host_cu),
                                                          _array_ptr(host_ctx))
        stream = _stream(k_cache.device)
        workspace = _decode_workspace(k_cache.device, stream, ws_bytes) if ws_bytes > 0 else None
        self._fn = lib.nie_varlen_prefill
        self._dtype = k_cache.dtype
        self._device = k_cache.device
        self._shape = (total_tokens, q_heads, head_dim)
        self._align = _row_align(q_heads, kv_heads, head_dim)
        self._keep = (cu_seqlens, context_lens, block_tables, workspace, host_cu, host_ctx)
        self._args = (dtype_code(k_cache.dtype), cu_seqlens.data_ptr(), context_lens.data_ptr(), num_seqs,
                      total_tokens, max_query_len, max_seq_len, k_cache.data_ptr(), v_cache.data_ptr(), num_layers,
                      num_blocks, block_size, q_heads, kv_heads, head_dim, block_tables.data_ptr(),
                      block_tables.shape[1], float(scale),
                      (None, 0) if workspace is None else (workspace.data_ptr(), workspace.numel()),
                      (_array_ptr(host_cu), _array_ptr(host_ctx)), stream)

    def __call__(self, query: torch.Tensor, layer_index: int, out: torch.Tensor) -> torch.Tensor:
        for t in (query, out):
            if (t.shape != self._shape or t.dtype != self._dtype or t.device != self._device or t.stride(2) != 1
                    or t.data_ptr() % self._align):
                raise ValueError("query/out must be aligned (tokens, q_heads, head_dim) tensors matching the batch")
        (code, cu, ctx, num_seqs, total, max_q, max_s, kptr, vptr, num_layers, num_blocks, block_size, q_heads,
         kv_heads, head_dim, tables, tstride, scale, (ws, ws_bytes), (hcu, hctx), stream) = self._args
        rc = self._fn(code, query.data_ptr(), query.stride(0), query.stride(1), cu, ctx, num_seqs, total, max_q,
                      max_s, kptr, vptr, num_layers, layer_index, num_blocks, block_size, q_heads, kv_heads, head_dim,
                      tables, tstride, scale, out.data_ptr(), out.stride(0), out.stride(1), ws, ws_bytes, hcu, hctx,
                      stream)
        if rc:
            _check(rc, "nie_varlen_prefill")
        return out
