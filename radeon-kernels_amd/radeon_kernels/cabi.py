"""ctypes binding of the C ABI in ``include/rk_paged_attention.h`` (``librk_pa_gfx950.so``).

This is the boundary a non-Python host (or a test) uses: plain device pointers, int64 sizes and a
HIP stream handle.  ``decode`` adapts torch tensors to it (allocating the output and split-K
workspace with torch on the current stream).  ``phase="fused"`` calls the single-launch entry,
whose arrival counters the caller keeps zeroed (they are left zero by every completed call).  Loading fails loudly if the library was not built;
there is no fallback here.

torch is imported before the library is opened so that the library binds to the HIP runtime torch
already loaded (both carry the soname ``libamdhip64.so.7``) instead of loading a second copy.
"""

from __future__ import annotations

import ctypes
import math
from pathlib import Path
from typing import Any

LIBRARY_PATH = Path(__file__).resolve().parents[1] / "packs" / "gfx950" / "lib" / "librk_pa_gfx950.so"

RK_OK = 0
RK_ERR_INVALID_ARGUMENT = 1
RK_ERR_UNSUPPORTED = 2
RK_ERR_WORKSPACE = 3
RK_ERR_LAUNCH = 4
RK_DTYPE_FP16 = 0
RK_DTYPE_BF16 = 1
RK_INDEX_INT32 = 0
RK_INDEX_INT64 = 1
RK_PA_NOALLOC_SCRATCH_BYTES = 32 * 1024 * 1024
VARIANTS = {"mfma": 0, "valu": 1, "mfma_qk": 2}
# Partition-kernel schedule bits OR-ed into the variant (RK_PA_SCHEDULE_*); "auto" lets the library
# choose.
SCHEDULES = {"auto": 0, "grid": 0x100, "queue": 0x200}
# Partition growth (RK_PA_PARTITION_GROW): partition_tokens is the smallest partition size the
# work-queue schedule runs.
RK_PA_PARTITION_GROW = 0x400

EXPORTED_SYMBOLS = (
    "rk_pa_decode",
    "rk_pa_decode_partitions",
    "rk_pa_decode_reduce",
    "rk_pa_decode_append",
    "rk_pa_decode_fused",
    "rk_pa_decode_counter_words",
    "rk_pa_decode_workspace_bytes",
    "rk_pa_decode_noalloc",
    "rk_pa_decode_schedule",
    "rk_pa_last_error",
    "rk_pa_version",
)
PHASES = {"all": "rk_pa_decode", "partitions": "rk_pa_decode_partitions", "reduce": "rk_pa_decode_reduce"}


def _variant_bits(variant: str, schedule: str, grow: bool) -> int:
    return VARIANTS[variant] | SCHEDULES[schedule] | (RK_PA_PARTITION_GROW if grow else 0)


def _repeatable(function: Any, args: tuple[Any, ...], check: Any, held: tuple[Any, ...]) -> Any:
    """A zero-argument callable repeating ``function(*args)`` (``check`` raises on a non-zero status).

    It keeps ``held`` -- the tensors the pointer arguments point into -- alive.
    """

    def launch(_held: tuple[Any, ...] = held) -> None:
        status = function(*args)
        if status:
            check(status)

    return launch


class CabiError(RuntimeError):
    def __init__(self, status: int, message: str) -> None:
        self.status = status
        super().__init__(f"rk_pa status {status}: {message}")


class PagedAttentionLibrary:
    def __init__(self, path: Path | str | None = None) -> None:
        import torch  # noqa: F401  (bind to torch's HIP runtime, see module docstring)

        self.path = Path(path) if path is not None else LIBRARY_PATH
        if not self.path.is_file():
            raise FileNotFoundError(
                f"native library {self.path} is missing; build it with `python radeon-kernels_amd/build.py`"
            )
        lib = ctypes.CDLL(str(self.path))
        i64, vp, sz = ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
        lib.rk_pa_decode_workspace_bytes.argtypes = [i64, i64, i64, i64, i64, i64, ctypes.POINTER(sz)]
        lib.rk_pa_decode_workspace_bytes.restype = ctypes.c_int
        decode_args = [vp, vp, vp, vp, vp, vp, vp, sz, i64, i64, i64, i64, i64, i64, i64,
                       ctypes.c_float, ctypes.c_int, ctypes.c_int, i64, ctypes.c_int, vp]
        for symbol in PHASES.values():
            getattr(lib, symbol).argtypes = decode_args
            getattr(lib, symbol).restype = ctypes.c_int
        lib.rk_pa_decode_fused.argtypes = decode_args[:8] + [vp, sz] + decode_args[8:]
        lib.rk_pa_decode_fused.restype = ctypes.c_int
        lib.rk_pa_decode_append.argtypes = [vp, vp, vp] + decode_args[1:8] + [vp, sz] + decode_args[8:]
        lib.rk_pa_decode_append.restype = ctypes.c_int
        lib.rk_pa_decode_noalloc.argtypes = decode_args[:6] + decode_args[8:]
        lib.rk_pa_decode_noalloc.restype = ctypes.c_int
        lib.rk_pa_decode_counter_words.argtypes = [i64, i64, i64, ctypes.POINTER(sz)]
        lib.rk_pa_decode_counter_words.restype = ctypes.c_int
        lib.rk_pa_decode_schedule.argtypes = [i64, i64, i64, i64, i64, i64, ctypes.c_int, i64, ctypes.c_int,
                                              ctypes.POINTER(ctypes.c_int)]
        lib.rk_pa_decode_schedule.restype = ctypes.c_int
        lib.rk_pa_last_error.argtypes = []
        lib.rk_pa_last_error.restype = ctypes.c_char_p
        lib.rk_pa_version.argtypes = []
        lib.rk_pa_version.restype = ctypes.c_char_p
        self.lib = lib

    def version(self) -> str:
        return self.lib.rk_pa_version().decode()

    def last_error(self) -> str:
        return self.lib.rk_pa_last_error().decode()

    def check(self, status: int) -> None:
        if status != RK_OK:
            raise CabiError(status, self.last_error())

    def schedule(self, batch: int, query_heads: int, kv_heads: int, head_dim: int, block_size: int,
                 max_blocks: int, dtype: str, partition_tokens: int, variant: str = "mfma",
                 schedule: str = "auto", grow: bool = False) -> str:
        """``"grid"`` or ``"queue"``: the partition-kernel schedule a decode with these arguments runs on
        the current device (rk_pa_decode_schedule)."""

        out = ctypes.c_int(0)
        self.check(self.lib.rk_pa_decode_schedule(batch, query_heads, kv_heads, head_dim, block_size, max_blocks,
                                                  RK_DTYPE_BF16 if dtype == "bf16" else RK_DTYPE_FP16,
                                                  partition_tokens, _variant_bits(variant, schedule, grow),
                                                  ctypes.byref(out)))
        return {SCHEDULES["grid"]: "grid", SCHEDULES["queue"]: "queue"}[out.value]

    def workspace_bytes(self, batch: int, query_heads: int, head_dim: int, block_size: int, max_blocks: int,
                        partition_tokens: int) -> int:
        out = ctypes.c_size_t(0)
        self.check(self.lib.rk_pa_decode_workspace_bytes(batch, query_heads, head_dim, block_size, max_blocks,
                                                         partition_tokens, ctypes.byref(out)))
        return int(out.value)

    def counter_words(self, batch: int, query_heads: int, kv_heads: int) -> int:
        out = ctypes.c_size_t(0)
        self.check(self.lib.rk_pa_decode_counter_words(batch, query_heads, kv_heads, ctypes.byref(out)))
        return int(out.value)

    def _raw_call(self, *, query: int, key_cache: int, value_cache: int, block_tables: int, context_lengths: int,
                  output: int, workspace: int, workspace_bytes: int, batch: int, query_heads: int, kv_heads: int,
                  head_dim: int, num_blocks: int, block_size: int, max_blocks: int, scale: float, dtype: int,
                  index_dtype: int, partition_tokens: int, variant: int, stream: int, phase: str = "all",
                  counters: int = 0, counter_words: int = 0, new_key: int = 0,
                  new_value: int = 0) -> tuple[Any, tuple[Any, ...]]:
        """The C entry point of ``phase`` and its argument tuple; with ``new_key`` / ``new_value``,
        rk_pa_decode_append in the two-launch (``"all"``) or single-launch (``"fused"``) form."""

        head = (query, key_cache, value_cache, block_tables, context_lengths, output, workspace or None,
                workspace_bytes)
        tail = (batch, query_heads, kv_heads, head_dim, num_blocks, block_size, max_blocks, ctypes.c_float(scale),
                dtype, index_dtype, partition_tokens, variant, stream or None)
        if new_key or new_value:
            if phase not in ("all", "fused"):
                raise ValueError("append-and-decode runs as phase 'all' or 'fused'")
            fused = phase == "fused"
            return self.lib.rk_pa_decode_append, (query, new_key or None, new_value or None, *head[1:],
                                                  (counters or None) if fused else None,
                                                  counter_words if fused else 0, *tail)
        if phase == "fused":
            return self.lib.rk_pa_decode_fused, (*head, counters or None, counter_words, *tail)
        return getattr(self.lib, PHASES[phase]), (*head, *tail)

    def decode_noalloc_raw(self, *, query: int, key_cache: int, value_cache: int, block_tables: int,
                           context_lengths: int, output: int, batch: int, query_heads: int, kv_heads: int,
                           head_dim: int, num_blocks: int, block_size: int, max_blocks: int, scale: float,
                           dtype: int, index_dtype: int, partition_tokens: int, variant: int, stream: int) -> int:
        """rk_pa_decode_noalloc on raw device pointers; returns the status."""

        return self.lib.rk_pa_decode_noalloc(query, key_cache, value_cache, block_tables, context_lengths, output,
                                             batch, query_heads, kv_heads, head_dim, num_blocks, block_size,
                                             max_blocks, ctypes.c_float(scale), dtype, index_dtype,
                                             partition_tokens, variant, stream or None)

    def decode_noalloc(self, query: Any, key_cache: Any, value_cache: Any, block_tables: Any, context_lengths: Any,
                       scale: float | None = None, *, out: Any, partition_tokens: int = 512, variant: str = "mfma",
                       stream: Any | None = None, schedule: str = "auto", grow: bool = False) -> Any:
        """rk_pa_decode_noalloc on torch tensors: writes ``out`` (caller-allocated) and returns it.

        The split-K records live in the library's per-GPU scratch array, so nothing is allocated
        here or in the library.
        """

        import torch

        batch, query_heads, head_dim = (int(s) for s in query.shape)
        num_blocks, block_size, kv_heads, _ = (int(s) for s in key_cache.shape)
        if scale is None:
            scale = 1.0 / math.sqrt(head_dim)
        if stream is None:
            stream = torch.cuda.current_stream(query.device)
        self.check(self.decode_noalloc_raw(
            query=query.data_ptr(), key_cache=key_cache.data_ptr(), value_cache=value_cache.data_ptr(),
            block_tables=block_tables.data_ptr(), context_lengths=context_lengths.data_ptr(), output=out.data_ptr(),
            batch=batch, query_heads=query_heads, kv_heads=kv_heads, head_dim=head_dim, num_blocks=num_blocks,
            block_size=block_size, max_blocks=int(block_tables.shape[1]), scale=float(scale),
            dtype=RK_DTYPE_BF16 if query.dtype == torch.bfloat16 else RK_DTYPE_FP16,
            index_dtype=RK_INDEX_INT64 if block_tables.dtype == torch.int64 else RK_INDEX_INT32,
            partition_tokens=partition_tokens, variant=_variant_bits(variant, schedule, grow),
            stream=stream.cuda_stream))
        return out

    def decode_raw(self, **arguments: Any) -> int:
        """One launch on raw device pointers (the keywords of ``_raw_call``); returns the status."""

        function, args = self._raw_call(**arguments)
        return function(*args)

    def _tensor_call(self, query: Any, key_cache: Any, value_cache: Any, block_tables: Any, context_lengths: Any,
                     scale: float | None, partition_tokens: int, variant: str, out: Any | None,
                     workspace: Any | None, stream: Any | None, phase: str, counters: Any | None,
                     new_key: Any | None = None, new_value: Any | None = None,
                     schedule: str = "auto", grow: bool = False) -> tuple[Any, Any, tuple[Any, ...], tuple[Any, ...]]:
        """(out, C function, its arguments, tensors those arguments point into)."""

        import torch

        batch, query_heads, head_dim = (int(s) for s in query.shape)
        num_blocks, block_size, kv_heads, _ = (int(s) for s in key_cache.shape)
        max_blocks = int(block_tables.shape[1])
        if scale is None:
            scale = 1.0 / math.sqrt(head_dim)
        need = self.workspace_bytes(batch, query_heads, head_dim, block_size, max_blocks, partition_tokens)
        if out is None:
            out = torch.empty_like(query)
        if need and workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=query.device)
        if stream is None:
            stream = torch.cuda.current_stream(query.device)
        if phase == "fused" and counters is None:
            counters = torch.zeros(self.counter_words(batch, query_heads, kv_heads), dtype=torch.int32,
                                   device=query.device)
        function, args = self._raw_call(
            query=query.data_ptr(), key_cache=key_cache.data_ptr(), value_cache=value_cache.data_ptr(),
            block_tables=block_tables.data_ptr(), context_lengths=context_lengths.data_ptr(), output=out.data_ptr(),
            workspace=workspace.data_ptr() if need else 0, workspace_bytes=workspace.numel() if need else 0,
            batch=batch, query_heads=query_heads, kv_heads=kv_heads, head_dim=head_dim, num_blocks=num_blocks,
            block_size=block_size, max_blocks=max_blocks, scale=float(scale),
            dtype=RK_DTYPE_BF16 if query.dtype == torch.bfloat16 else RK_DTYPE_FP16,
            index_dtype=RK_INDEX_INT64 if block_tables.dtype == torch.int64 else RK_INDEX_INT32,
            partition_tokens=partition_tokens, variant=_variant_bits(variant, schedule, grow),
            stream=stream.cuda_stream, phase=phase,
            counters=counters.data_ptr() if counters is not None else 0,
            counter_words=counters.numel() if counters is not None else 0,
            new_key=new_key.data_ptr() if new_key is not None else 0,
            new_value=new_value.data_ptr() if new_value is not None else 0,
        )
        held = (query, key_cache, value_cache, block_tables, context_lengths, out, workspace, counters, new_key,
                new_value)
        return out, function, args, held

    def decode(self, query: Any, key_cache: Any, value_cache: Any, block_tables: Any, context_lengths: Any,
               scale: float | None = None, *, partition_tokens: int = 512, variant: str = "mfma",
               out: Any | None = None, workspace: Any | None = None, stream: Any | None = None,
               phase: str = "all", counters: Any | None = None, new_key: Any | None = None,
               new_value: Any | None = None, schedule: str = "auto", grow: bool = False) -> Any:
        """Launch on torch tensors (all on one GPU); returns ``out`` (allocated if None).

        ``counters`` (phase ``"fused"`` only): an int32 tensor of at least ``counter_words`` zeros,
        allocated zeroed here if None.  ``new_key`` / ``new_value`` ([batch, kv_heads, head_dim]):
        append-and-decode (rk_pa_decode_append), which also writes them into the caches.
        ``schedule``: ``"auto"``, ``"grid"`` or ``"queue"`` (the RK_PA_SCHEDULE_* bits); ``grow``:
        partition growth (RK_PA_PARTITION_GROW).
        """

        out, function, args, _ = self._tensor_call(query, key_cache, value_cache, block_tables, context_lengths,
                                                   scale, partition_tokens, variant, out, workspace, stream, phase,
                                                   counters, new_key, new_value, schedule, grow)
        self.check(function(*args))
        return out

    def prepare(self, query: Any, key_cache: Any, value_cache: Any, block_tables: Any, context_lengths: Any,
                scale: float | None = None, *, partition_tokens: int = 512, variant: str = "mfma",
                out: Any | None = None, workspace: Any | None = None, stream: Any | None = None,
                phase: str = "all", counters: Any | None = None, new_key: Any | None = None,
                new_value: Any | None = None, schedule: str = "auto", grow: bool = False) -> Any:
        """The launch ``decode`` would make, with every argument converted once.

        Returns a zero-argument callable that repeats it (one foreign call per launch, no Python
        shape handling): what a timing loop needs to measure the GPU rather than this wrapper.  The
        callable keeps the tensors it points into alive.
        """

        _, function, args, held = self._tensor_call(query, key_cache, value_cache, block_tables, context_lengths,
                                                    scale, partition_tokens, variant, out, workspace, stream,
                                                    phase, counters, new_key, new_value, schedule, grow)
        return _repeatable(function, args, self.check, held)


_LIBRARY: PagedAttentionLibrary | None = None


def library() -> PagedAttentionLibrary:
    global _LIBRARY
    if _LIBRARY is None:
        _LIBRARY = PagedAttentionLibrary()
    return _LIBRARY


# ---------------------------------------------------------------------------------------------
# Paged KV-cache library (include/rk_kv_cache.h).
KV_LIBRARY_PATH = LIBRARY_PATH.parent / "librk_kv_gfx950.so"
KV_EXPORTED_SYMBOLS = ("rk_kv_cache_append", "rk_kv_cache_copy", "rk_kv_last_error", "rk_kv_version")
RK_KV_OK = 0
RK_KV_ERR_INVALID_ARGUMENT = 1
RK_KV_ERR_UNSUPPORTED = 2
RK_KV_ERR_LAUNCH = 4


class KvCacheLibrary:
    def __init__(self, path: Path | str | None = None) -> None:
        import torch  # noqa: F401  (bind to torch's HIP runtime, see module docstring)

        self.path = Path(path) if path is not None else KV_LIBRARY_PATH
        if not self.path.is_file():
            raise FileNotFoundError(
                f"native library {self.path} is missing; build it with `python radeon-kernels_amd/build.py`"
            )
        lib = ctypes.CDLL(str(self.path))
        i64, vp = ctypes.c_int64, ctypes.c_void_p
        lib.rk_kv_cache_append.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int, ctypes.c_int, vp]
        lib.rk_kv_cache_append.restype = ctypes.c_int
        lib.rk_kv_cache_copy.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int, ctypes.c_int, vp]
        lib.rk_kv_cache_copy.restype = ctypes.c_int
        lib.rk_kv_last_error.argtypes = []
        lib.rk_kv_last_error.restype = ctypes.c_char_p
        lib.rk_kv_version.argtypes = []
        lib.rk_kv_version.restype = ctypes.c_char_p
        self.lib = lib

    def version(self) -> str:
        return self.lib.rk_kv_version().decode()

    def last_error(self) -> str:
        return self.lib.rk_kv_last_error().decode()

    def append_raw(self, *, key: int, value: int, key_cache: int, value_cache: int, slot_mapping: int, tokens: int,
                   kv_heads: int, head_dim: int, num_blocks: int, block_size: int, dtype: int, index_dtype: int,
                   stream: int) -> int:
        return self.lib.rk_kv_cache_append(key, value, key_cache, value_cache, slot_mapping, tokens, kv_heads,
                                           head_dim, num_blocks, block_size, dtype, index_dtype, stream or None)

    def check(self, status: int) -> None:
        if status != RK_KV_OK:
            raise CabiError(status, self.last_error())

    def _append_call(self, key: Any, value: Any, key_cache: Any, value_cache: Any, slot_mapping: Any,
                     stream: Any | None) -> tuple[Any, tuple[Any, ...]]:
        import torch

        tokens, kv_heads, head_dim = (int(s) for s in key.shape)
        num_blocks, block_size = int(key_cache.shape[0]), int(key_cache.shape[1])
        if stream is None:
            stream = torch.cuda.current_stream(key.device)
        return self.lib.rk_kv_cache_append, (
            key.data_ptr(), value.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), slot_mapping.data_ptr(),
            tokens, kv_heads, head_dim, num_blocks, block_size,
            RK_DTYPE_BF16 if key.dtype == torch.bfloat16 else RK_DTYPE_FP16,
            RK_INDEX_INT64 if slot_mapping.dtype == torch.int64 else RK_INDEX_INT32, stream.cuda_stream or None)

    def append(self, key: Any, value: Any, key_cache: Any, value_cache: Any, slot_mapping: Any, *,
               stream: Any | None = None) -> tuple[Any, Any]:
        """Launch on torch tensors (all on one GPU); writes the caches in place and returns them."""

        function, args = self._append_call(key, value, key_cache, value_cache, slot_mapping, stream)
        self.check(function(*args))
        return key_cache, value_cache

    def prepare_append(self, key: Any, value: Any, key_cache: Any, value_cache: Any, slot_mapping: Any, *,
                       stream: Any | None = None) -> Any:
        """``append``'s launch with its arguments converted once; calling the result repeats it."""

        function, args = self._append_call(key, value, key_cache, value_cache, slot_mapping, stream)
        return _repeatable(function, args, self.check, (key, value, key_cache, value_cache, slot_mapping))

    def copy_raw(self, *, key_cache: int, value_cache: int, block_mapping: int, pairs: int, num_blocks: int,
                 block_size: int, kv_heads: int, head_dim: int, dtype: int, index_dtype: int, stream: int) -> int:
        return self.lib.rk_kv_cache_copy(key_cache, value_cache, block_mapping, pairs, num_blocks, block_size,
                                         kv_heads, head_dim, dtype, index_dtype, stream or None)

    def _copy_call(self, key_cache: Any, value_cache: Any, block_mapping: Any,
                   stream: Any | None) -> tuple[Any, tuple[Any, ...]]:
        import torch

        num_blocks, block_size, kv_heads, head_dim = (int(s) for s in key_cache.shape)
        if stream is None:
            stream = torch.cuda.current_stream(key_cache.device)
        return self.lib.rk_kv_cache_copy, (
            key_cache.data_ptr(), value_cache.data_ptr(), block_mapping.data_ptr(), int(block_mapping.shape[0]),
            num_blocks, block_size, kv_heads, head_dim,
            RK_DTYPE_BF16 if key_cache.dtype == torch.bfloat16 else RK_DTYPE_FP16,
            RK_INDEX_INT64 if block_mapping.dtype == torch.int64 else RK_INDEX_INT32, stream.cuda_stream or None)

    def copy(self, key_cache: Any, value_cache: Any, block_mapping: Any, *, stream: Any | None = None
             ) -> tuple[Any, Any]:
        """Launch on torch tensors (all on one GPU); copies blocks in place and returns the caches."""

        function, args = self._copy_call(key_cache, value_cache, block_mapping, stream)
        self.check(function(*args))
        return key_cache, value_cache

    def prepare_copy(self, key_cache: Any, value_cache: Any, block_mapping: Any, *,
                     stream: Any | None = None) -> Any:
        """``copy``'s launch with its arguments converted once; calling the result repeats it."""

        function, args = self._copy_call(key_cache, value_cache, block_mapping, stream)
        return _repeatable(function, args, self.check, (key_cache, value_cache, block_mapping))


_KV_LIBRARY: KvCacheLibrary | None = None


def kv_library() -> KvCacheLibrary:
    global _KV_LIBRARY
    if _KV_LIBRARY is None:
        _KV_LIBRARY = KvCacheLibrary()
    return _KV_LIBRARY


# ---------------------------------------------------------------------------------------------
# Self-attention library (include/rk_sdpa.h).
SDPA_LIBRARY_PATH = LIBRARY_PATH.parent / "librk_sdpa_gfx950.so"
SDPA_EXPORTED_SYMBOLS = ("rk_sdpa_forward", "rk_sdpa_last_error", "rk_sdpa_version")
RK_SDPA_OK = 0
RK_SDPA_ERR_INVALID_ARGUMENT = 1
RK_SDPA_ERR_UNSUPPORTED = 2
RK_SDPA_ERR_LAUNCH = 4


class SdpaLibrary:
    """ctypes binding of ``librk_sdpa_gfx950.so``; ``forward`` adapts torch tensors to it."""

    def __init__(self, path: Path | str | None = None) -> None:
        import torch  # noqa: F401  (bind to torch's HIP runtime, see module docstring)

        self.path = Path(path) if path is not None else SDPA_LIBRARY_PATH
        if not self.path.is_file():
            raise FileNotFoundError(
                f"native library {self.path} is missing; build it with `python radeon-kernels_amd/build.py`")
        lib = ctypes.CDLL(str(self.path))
        i64, vp = ctypes.c_int64, ctypes.c_void_p
        lib.rk_sdpa_forward.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int, ctypes.c_float,
                                        ctypes.c_int, vp]
        lib.rk_sdpa_forward.restype = ctypes.c_int
        lib.rk_sdpa_last_error.argtypes = []
        lib.rk_sdpa_last_error.restype = ctypes.c_char_p
        lib.rk_sdpa_version.argtypes = []
        lib.rk_sdpa_version.restype = ctypes.c_char_p
        self.lib = lib

    def version(self) -> str:
        return self.lib.rk_sdpa_version().decode()

    def last_error(self) -> str:
        return self.lib.rk_sdpa_last_error().decode()

    def forward_raw(self, *, query: int, key: int, value: int, output: int, batch: int, query_heads: int,
                    kv_heads: int, sequence: int, head_dim: int, is_causal: int, scale: float, dtype: int,
                    stream: int) -> int:
        return self.lib.rk_sdpa_forward(query, key, value, output, batch, query_heads, kv_heads, sequence, head_dim,
                                        is_causal, ctypes.c_float(scale), dtype, stream or None)

    def check(self, status: int) -> None:
        if status != RK_SDPA_OK:
            raise CabiError(status, self.last_error())

    def _forward_call(self, query: Any, key: Any, value: Any, is_causal: bool, scale: float | None,
                      out: Any | None, stream: Any | None) -> tuple[Any, Any, tuple[Any, ...]]:
        import torch

        batch, query_heads, sequence, head_dim = (int(s) for s in query.shape)
        if scale is None:
            scale = 1.0 / math.sqrt(head_dim)
        if out is None:
            out = torch.empty_like(query)
        if stream is None:
            stream = torch.cuda.current_stream(query.device)
        return out, self.lib.rk_sdpa_forward, (
            query.data_ptr(), key.data_ptr(), value.data_ptr(), out.data_ptr(), batch, query_heads, int(key.shape[1]),
            sequence, head_dim, int(bool(is_causal)), ctypes.c_float(float(scale)),
            RK_DTYPE_BF16 if query.dtype == torch.bfloat16 else RK_DTYPE_FP16, stream.cuda_stream or None)

    def forward(self, query: Any, key: Any, value: Any, *, is_causal: bool = False, scale: float | None = None,
                out: Any | None = None, stream: Any | None = None) -> Any:
        out, function, args = self._forward_call(query, key, value, is_causal, scale, out, stream)
        self.check(function(*args))
        return out

    def prepare_forward(self, query: Any, key: Any, value: Any, *, is_causal: bool = False,
                        scale: float | None = None, out: Any | None = None, stream: Any | None = None) -> Any:
        """``forward``'s launch with its arguments converted once; calling the result repeats it."""

        out, function, args = self._forward_call(query, key, value, is_causal, scale, out, stream)
        return _repeatable(function, args, self.check, (query, key, value, out))


_SDPA_LIBRARY: SdpaLibrary | None = None


def sdpa_library() -> SdpaLibrary:
    global _SDPA_LIBRARY
    if _SDPA_LIBRARY is None:
        _SDPA_LIBRARY = SdpaLibrary()
    return _SDPA_LIBRARY
