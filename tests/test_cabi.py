"""CPU tests of the C ABI (include/rk_paged_attention.h) without launching anything.

* The built library loads and exports every function the header declares.
* Workspace sizing follows the documented formula.
* Invalid arguments are rejected with the documented status codes and messages before any launch
  (every call here fails validation, so no device memory is touched and no GPU is needed).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from radeon_kernels import cabi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "rk_paged_attention.h"


@pytest.fixture(scope="module")
def lib():
    if not cabi.LIBRARY_PATH.is_file():
        pytest.fail(f"{cabi.LIBRARY_PATH} is not built; run __graft_entry__.build()")
    return cabi.PagedAttentionLibrary()


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(rk_\w+)\s*\(", text, flags=re.MULTILINE)))


def test_header_declares_the_documented_entry_points():
    assert declared_functions() == sorted(cabi.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib.lib, name), name
    assert lib.version() == "rk_pa_gfx950 1.0.0 (gfx950, wave64)"


def test_append_and_decode_argument_assembly(lib):
    """rk_pa_decode_append takes the new rows after the query and the counters only in the fused
    form; the split phases cannot carry an append (no call reaches the device here)."""

    shape = dict(query=0x1000, key_cache=0x2000, value_cache=0x3000, block_tables=0x4000, context_lengths=0x5000,
                 output=0x6000, workspace=0x7000, workspace_bytes=256, batch=2, query_heads=8, kv_heads=2,
                 head_dim=128, num_blocks=4, block_size=16, max_blocks=2, scale=0.125, dtype=cabi.RK_DTYPE_BF16,
                 index_dtype=cabi.RK_INDEX_INT32, partition_tokens=16, variant=cabi.VARIANTS["mfma"], stream=0,
                 counters=0x8000, counter_words=4, new_key=0x9000, new_value=0xA000)
    function, args = lib._raw_call(**shape, phase="all")
    assert function == lib.lib.rk_pa_decode_append
    assert args[:4] == (0x1000, 0x9000, 0xA000, 0x2000) and args[10:12] == (None, 0)
    function, args = lib._raw_call(**shape, phase="fused")
    assert function == lib.lib.rk_pa_decode_append and args[10:12] == (0x8000, 4)
    for phase in ("partitions", "reduce"):
        with pytest.raises(ValueError):
            lib._raw_call(**shape, phase=phase)
    function, _ = lib._raw_call(**{**shape, "new_key": 0, "new_value": 0}, phase="all")
    assert function == lib.lib.rk_pa_decode


def test_status_codes_match_header():
    text = HEADER.read_text()
    for name in ("RK_OK", "RK_ERR_INVALID_ARGUMENT", "RK_ERR_UNSUPPORTED", "RK_ERR_WORKSPACE", "RK_ERR_LAUNCH",
                 "RK_DTYPE_FP16", "RK_DTYPE_BF16", "RK_INDEX_INT32", "RK_INDEX_INT64"):
        value = int(re.search(rf"#define {name} (\d+)", text).group(1))
        assert getattr(cabi, name) == value, name
    assert cabi.VARIANTS == {"mfma": int(re.search(r"RK_PA_VARIANT_MFMA (\d+)", text).group(1)),
                             "valu": int(re.search(r"RK_PA_VARIANT_VALU (\d+)", text).group(1)),
                             "mfma_qk": int(re.search(r"RK_PA_VARIANT_MFMA_QK (\d+)", text).group(1))}
    assert cabi.SCHEDULES == {"auto": 0, "grid": int(re.search(r"RK_PA_SCHEDULE_GRID (0x[0-9a-f]+)", text).group(1), 16),
                              "queue": int(re.search(r"RK_PA_SCHEDULE_QUEUE (0x[0-9a-f]+)", text).group(1), 16)}
    assert cabi.RK_PA_PARTITION_GROW == int(re.search(r"RK_PA_PARTITION_GROW (0x[0-9a-f]+)", text).group(1), 16)


def expected_workspace(batch, hq, d, bs, mb, partition):
    """256-byte work-queue header, accumulator records padded to 256 B, then (max, sum) pairs."""

    parts = -(-(mb * bs) // partition)
    if parts <= 1:
        return 0
    records = batch * hq * parts
    return 256 + ((records * d * 4 + 255) // 256) * 256 + records * 2 * 4


@pytest.mark.parametrize("shape", [(128, 32, 128, 16, 1024, 2048), (8, 32, 128, 16, 64, 64), (1, 32, 128, 16, 8, 128),
                                   (4, 16, 64, 32, 64, 128), (3, 12, 256, 1, 700, 256)])
def test_workspace_size_formula(lib, shape):
    assert lib.workspace_bytes(*shape) == expected_workspace(*shape)


def no_visible_gpu() -> bool:
    import torch

    return not torch.cuda.is_available()


# The calls below pass fake device pointers; each one must fail validation before any launch.  They
# are skipped where a GPU is visible so that a validation bug could never turn into a launch with
# invalid pointers.
cpu_only = pytest.mark.skipif(not no_visible_gpu(), reason="fake-pointer validation checks run without a GPU only")


def call(lib, **overrides):
    args = dict(query=16, key_cache=32, value_cache=48, block_tables=64, context_lengths=80, output=96, workspace=0,
                workspace_bytes=0, batch=2, query_heads=8, kv_heads=2, head_dim=128, num_blocks=8, block_size=16,
                max_blocks=4, scale=0.125, dtype=cabi.RK_DTYPE_BF16, index_dtype=cabi.RK_INDEX_INT32,
                partition_tokens=64, variant=0, stream=0)
    args.update(overrides)
    status = lib.decode_raw(**args)
    return status, lib.last_error()


@pytest.mark.parametrize(
    "overrides, status, message",
    [
        (dict(query=0), cabi.RK_ERR_INVALID_ARGUMENT, "must not be NULL"),
        (dict(dtype=7), cabi.RK_ERR_INVALID_ARGUMENT, "dtype"),
        (dict(index_dtype=3), cabi.RK_ERR_INVALID_ARGUMENT, "index_dtype"),
        (dict(variant=9), cabi.RK_ERR_INVALID_ARGUMENT, "variant"),
        (dict(scale=0.0), cabi.RK_ERR_INVALID_ARGUMENT, "positive and finite"),
        (dict(scale=float("inf")), cabi.RK_ERR_INVALID_ARGUMENT, "positive and finite"),
        (dict(query=24), cabi.RK_ERR_UNSUPPORTED, "16-byte aligned"),
        (dict(head_dim=80), cabi.RK_ERR_INVALID_ARGUMENT, "one of 64, 128, 256"),
        (dict(query_heads=9), cabi.RK_ERR_INVALID_ARGUMENT, "divisible by kv_heads"),
        (dict(block_size=48), cabi.RK_ERR_UNSUPPORTED, "power of two"),
        (dict(block_size=512), cabi.RK_ERR_UNSUPPORTED, "power of two"),
        (dict(partition_tokens=40), cabi.RK_ERR_INVALID_ARGUMENT, "multiple of 16"),
        (dict(partition_tokens=8192 * 2), cabi.RK_ERR_INVALID_ARGUMENT, "multiple of 16"),
        (dict(partition_tokens=8192, block_size=8), cabi.RK_ERR_INVALID_ARGUMENT, "<= 512"),
        (dict(batch=0), cabi.RK_ERR_INVALID_ARGUMENT, "positive"),
        (dict(num_blocks=1 << 31), cabi.RK_ERR_UNSUPPORTED, "32-bit"),
        (dict(kv_heads=1 << 19, query_heads=1 << 19), cabi.RK_ERR_UNSUPPORTED, "too large"),
        (dict(max_blocks=64, partition_tokens=64), cabi.RK_ERR_WORKSPACE, "workspace of"),
        (dict(max_blocks=64, partition_tokens=64, workspace=4096 + 64, workspace_bytes=1 << 20), cabi.RK_ERR_WORKSPACE,
         "256-byte aligned"),
        # Schedule bits: both at once, or an unknown bit, are invalid; the queue needs the MFMA variant,
        # a split-K shape (several partitions), at most 256 partitions and at most 64512 sequences
        # (launches of 1024).
        (dict(variant=0x300), cabi.RK_ERR_INVALID_ARGUMENT, "variant"),
        (dict(variant=0x800), cabi.RK_ERR_INVALID_ARGUMENT, "variant"),
        (dict(variant=0x700), cabi.RK_ERR_INVALID_ARGUMENT, "variant"),
        # Partition growth combines with either schedule and either variant; a forced queue still
        # needs an eligible shape, and the workspace is that of partition_tokens.
        (dict(variant=0x600), cabi.RK_ERR_UNSUPPORTED, "work-queue schedule"),
        (dict(variant=0x401, max_blocks=64), cabi.RK_ERR_WORKSPACE, "workspace of"),
        (dict(variant=0x500, max_blocks=64, workspace=1 << 20, workspace_bytes=100), cabi.RK_ERR_WORKSPACE,
         "workspace of"),
        (dict(variant=0x201, max_blocks=64, workspace=1 << 20, workspace_bytes=1 << 20), cabi.RK_ERR_UNSUPPORTED,
         "work-queue schedule"),
        (dict(variant=0x200), cabi.RK_ERR_UNSUPPORTED, "work-queue schedule"),
        (dict(variant=0x200, max_blocks=1024, partition_tokens=16, workspace=1 << 20, workspace_bytes=1 << 30),
         cabi.RK_ERR_UNSUPPORTED, "work-queue schedule"),
        (dict(variant=0x200, batch=64513, max_blocks=64, workspace=1 << 20, workspace_bytes=1 << 40),
         cabi.RK_ERR_UNSUPPORTED, "work-queue schedule"),
    ],
)
@cpu_only
def test_invalid_arguments_are_rejected_before_launch(lib, overrides, status, message):
    got, text = call(lib, **overrides)
    assert got == status, text
    assert message in text


@pytest.mark.parametrize(
    "overrides, status, message",
    [
        (dict(dtype=5), cabi.RK_ERR_INVALID_ARGUMENT, "dtype"),
        (dict(variant=0x300), cabi.RK_ERR_INVALID_ARGUMENT, "variant"),
        (dict(variant=7), cabi.RK_ERR_INVALID_ARGUMENT, "variant"),
        (dict(head_dim=96), cabi.RK_ERR_INVALID_ARGUMENT, "one of 64, 128, 256"),
        (dict(variant=0x200, max_blocks=4), cabi.RK_ERR_UNSUPPORTED, "work-queue schedule"),
        (dict(variant=0x201), cabi.RK_ERR_UNSUPPORTED, "work-queue schedule"),
        (dict(variant=0x601), cabi.RK_ERR_UNSUPPORTED, "work-queue schedule"),
        (dict(variant=0xB00), cabi.RK_ERR_INVALID_ARGUMENT, "variant"),
    ],
)
def test_schedule_query_validates_before_asking_the_device(lib, overrides, status, message):
    """rk_pa_decode_schedule rejects what a decode would reject, before any runtime query."""

    args = dict(batch=8, query_heads=32, kv_heads=8, head_dim=128, block_size=16, max_blocks=64, dtype=1,
                partition_tokens=256, variant=0)
    args.update(overrides)
    out = ctypes.c_int(-1)
    got = lib.lib.rk_pa_decode_schedule(*args.values(), ctypes.byref(out))
    assert got == status, lib.last_error()
    assert message in lib.last_error()
    assert out.value == -1
    assert lib.lib.rk_pa_decode_schedule(8, 32, 8, 128, 16, 64, 1, 256, 0, None) == cabi.RK_ERR_INVALID_ARGUMENT


@cpu_only
def test_phase_entry_points_validate_identically(lib):
    for phase in ("partitions", "reduce"):
        status = lib.decode_raw(query=0, key_cache=32, value_cache=48, block_tables=64, context_lengths=80, output=96,
                                workspace=0, workspace_bytes=0, batch=2, query_heads=8, kv_heads=2, head_dim=128,
                                num_blocks=8, block_size=16, max_blocks=4, scale=0.125, dtype=1, index_dtype=0,
                                partition_tokens=64, variant=0, stream=0, phase=phase)
        assert status == cabi.RK_ERR_INVALID_ARGUMENT and "NULL" in lib.last_error()


def test_counter_words_formula(lib):
    """One arrival counter per (sequence, KV head, chunk of 1, 2 or 4 query heads) -- an upper bound for
    the 8-head chunks groups of 8 or more run at head_dim <= 128 -- then the work queue's ticket and
    exit counters."""

    for batch, hq, hkv, arrivals in [(128, 32, 8, 128 * 8), (3, 64, 8, 3 * 8 * 2), (2, 12, 4, 2 * 4),
                                     (5, 8, 8, 40), (1, 16, 8, 8), (2, 40, 8, 2 * 8 * 2)]:
        assert lib.counter_words(batch, hq, hkv) == arrivals + 2
    out = ctypes.c_size_t(0)
    assert lib.lib.rk_pa_decode_counter_words(1, 8, 2, None) == cabi.RK_ERR_INVALID_ARGUMENT
    assert lib.lib.rk_pa_decode_counter_words(1, 9, 2, ctypes.byref(out)) == cabi.RK_ERR_INVALID_ARGUMENT
    assert lib.lib.rk_pa_decode_counter_words(0, 8, 2, ctypes.byref(out)) == cabi.RK_ERR_INVALID_ARGUMENT


@cpu_only
@pytest.mark.parametrize(
    "overrides, status, message",
    [
        (dict(counters=0, counter_words=0), cabi.RK_ERR_WORKSPACE, "counter words required"),
        (dict(counters=4096, counter_words=5), cabi.RK_ERR_WORKSPACE, "6 counter words required, 5 given"),
        (dict(counters=4098, counter_words=64), cabi.RK_ERR_WORKSPACE, "4-byte aligned"),
        (dict(query=0), cabi.RK_ERR_INVALID_ARGUMENT, "must not be NULL"),
        (dict(workspace=0, workspace_bytes=0), cabi.RK_ERR_WORKSPACE, "workspace of"),
    ],
)
def test_fused_entry_validates_counters_before_launch(lib, overrides, status, message):
    # batch 2, 8 query heads over 2 KV heads (one chunk of 4) -> 4 arrival counters and the queue's 2; 4
    # partitions of 64 tokens.
    args = dict(phase="fused", max_blocks=16, workspace=1 << 20, workspace_bytes=1 << 20, counters=4096,
                counter_words=64)
    args.update(overrides)
    got, text = call(lib, **args)
    assert got == status, text
    assert message in text


@cpu_only
def test_last_error_is_per_thread(lib):
    import threading

    call(lib, dtype=7)
    seen = {}

    def worker():
        call(lib, variant=9)
        seen["thread"] = lib.last_error()

    thread = threading.Thread(target=worker)
    thread.start()
    thread.join()
    assert "variant" in seen["thread"]
    assert "dtype" in lib.last_error()


def test_noalloc_scratch_limit_matches_header():
    text = HEADER.read_text()
    match = re.search(r"#define RK_PA_NOALLOC_SCRATCH_BYTES \((\d+)u \* 1024u \* 1024u\)", text)
    assert match and int(match.group(1)) * 1024 * 1024 == cabi.RK_PA_NOALLOC_SCRATCH_BYTES


def noalloc_call(lib, **overrides):
    args = dict(query=16, key_cache=32, value_cache=48, block_tables=64, context_lengths=80, output=96, batch=2,
                query_heads=8, kv_heads=2, head_dim=128, num_blocks=8, block_size=16, max_blocks=4, scale=0.125,
                dtype=cabi.RK_DTYPE_BF16, index_dtype=cabi.RK_INDEX_INT32, partition_tokens=64, variant=0, stream=0)
    args.update(overrides)
    return lib.decode_noalloc_raw(**args), lib.last_error()


@cpu_only
@pytest.mark.parametrize(
    "overrides, status, message",
    [
        (dict(query=0), cabi.RK_ERR_INVALID_ARGUMENT, "must not be NULL"),
        (dict(dtype=7), cabi.RK_ERR_INVALID_ARGUMENT, "dtype"),
        (dict(head_dim=100), cabi.RK_ERR_INVALID_ARGUMENT, "head_dim"),
        (dict(partition_tokens=24), cabi.RK_ERR_INVALID_ARGUMENT, "partition_tokens"),
        # 4096 x 32 heads x 64 partitions of 16 tokens: 4096*32*64*(128+2)*4 bytes of records > 32 MiB.
        (dict(batch=4096, query_heads=32, kv_heads=8, max_blocks=64, partition_tokens=16), cabi.RK_ERR_WORKSPACE,
         "bytes of split-K scratch; rk_pa_decode_noalloc holds 33554432"),
    ],
)
def test_noalloc_validates_like_decode_before_any_device_call(lib, overrides, status, message):
    got, text = noalloc_call(lib, **overrides)
    assert got == status, text
    assert message in text


@cpu_only
def test_noalloc_scratch_limit_boundary(lib):
    """The largest shape whose records fit is accepted by validation (it then needs a device: without
    one the scratch lookup fails as a launch error); one more sequence is rejected."""

    # records of b sequences x 32 heads x 16 partitions (P 64 over 1024 tokens): b*32*16*(128*4) + b*32*16*8
    per_seq = 32 * 16 * 128 * 4 + 32 * 16 * 8
    fit = cabi.RK_PA_NOALLOC_SCRATCH_BYTES // per_seq
    assert lib.workspace_bytes(fit, 32, 128, 16, 64, 64) <= cabi.RK_PA_NOALLOC_SCRATCH_BYTES
    assert lib.workspace_bytes(fit + 1, 32, 128, 16, 64, 64) > cabi.RK_PA_NOALLOC_SCRATCH_BYTES
    got, text = noalloc_call(lib, batch=fit + 1, query_heads=32, kv_heads=8, max_blocks=64)
    assert got == cabi.RK_ERR_WORKSPACE, text
    got, text = noalloc_call(lib, batch=fit, query_heads=32, kv_heads=8, max_blocks=64)
    assert got == cabi.RK_ERR_LAUNCH and "hipGetDevice" in text, text


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(FileNotFoundError, match="build"):
        cabi.PagedAttentionLibrary(tmp_path / "absent.so")


def test_workspace_null_pointer_rejected(lib):
    out = ctypes.c_size_t(0)
    assert lib.lib.rk_pa_decode_workspace_bytes(1, 8, 128, 16, 4, 64, None) == cabi.RK_ERR_INVALID_ARGUMENT
    assert lib.lib.rk_pa_decode_workspace_bytes(1, 8, 128, 16, 4, 64, ctypes.byref(out)) == cabi.RK_OK


# ---------------------------------------------------------------------------------------------
# Paged KV-cache library (include/rk_kv_cache.h).
KV_HEADER = ROOT / "include" / "rk_kv_cache.h"


@pytest.fixture(scope="module")
def kvlib():
    if not cabi.KV_LIBRARY_PATH.is_file():
        pytest.fail(f"{cabi.KV_LIBRARY_PATH} is not built; run __graft_entry__.build()")
    return cabi.KvCacheLibrary()


def test_kv_header_and_library_agree(kvlib):
    text = KV_HEADER.read_text()
    declared = sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(rk_\w+)\s*\(", text, flags=re.MULTILINE)))
    assert declared == sorted(cabi.KV_EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(kvlib.lib, name), name
    for name in ("RK_KV_OK", "RK_KV_ERR_INVALID_ARGUMENT", "RK_KV_ERR_UNSUPPORTED", "RK_KV_ERR_LAUNCH"):
        assert getattr(cabi, name) == int(re.search(rf"#define {name} (\d+)", text).group(1)), name
    # Element-type codes are shared with the decode library.
    assert int(re.search(r"#define RK_KV_DTYPE_BF16 (\d+)", text).group(1)) == cabi.RK_DTYPE_BF16
    assert int(re.search(r"#define RK_KV_INDEX_INT64 (\d+)", text).group(1)) == cabi.RK_INDEX_INT64
    assert kvlib.version() == "rk_kv_gfx950 1.0.0 (gfx950, wave64)"


def kv_call(lib, **overrides):
    args = dict(key=16, value=32, key_cache=48, value_cache=64, slot_mapping=80, tokens=4, kv_heads=8, head_dim=128,
                num_blocks=16, block_size=16, dtype=cabi.RK_DTYPE_BF16, index_dtype=cabi.RK_INDEX_INT64, stream=0)
    args.update(overrides)
    return lib.append_raw(**args), lib.last_error()


@pytest.mark.parametrize(
    "overrides, status, message",
    [
        (dict(key=0), cabi.RK_KV_ERR_INVALID_ARGUMENT, "must not be NULL"),
        (dict(slot_mapping=0), cabi.RK_KV_ERR_INVALID_ARGUMENT, "must not be NULL"),
        (dict(dtype=5), cabi.RK_KV_ERR_INVALID_ARGUMENT, "dtype"),
        (dict(index_dtype=2), cabi.RK_KV_ERR_INVALID_ARGUMENT, "index_dtype"),
        (dict(tokens=0), cabi.RK_KV_ERR_INVALID_ARGUMENT, "positive"),
        (dict(block_size=-1), cabi.RK_KV_ERR_INVALID_ARGUMENT, "positive"),
        (dict(value=40), cabi.RK_KV_ERR_UNSUPPORTED, "16-byte aligned"),
        (dict(kv_heads=1, head_dim=7), cabi.RK_KV_ERR_UNSUPPORTED, "multiple of 16 bytes"),
        (dict(tokens=1 << 24, kv_heads=32, head_dim=128), cabi.RK_KV_ERR_UNSUPPORTED, "index range"),
    ],
)
@cpu_only
def test_kv_invalid_arguments_are_rejected_before_launch(kvlib, overrides, status, message):
    got, text = kv_call(kvlib, **overrides)
    assert got == status, text
    assert message in text


def test_kv_missing_library_fails_loudly(tmp_path):
    with pytest.raises(FileNotFoundError, match="build"):
        cabi.KvCacheLibrary(tmp_path / "absent.so")


def kv_copy_call(lib, **overrides):
    args = dict(key_cache=48, value_cache=64, block_mapping=80, pairs=4, num_blocks=16, block_size=16, kv_heads=8,
                head_dim=128, dtype=cabi.RK_DTYPE_BF16, index_dtype=cabi.RK_INDEX_INT64, stream=0)
    args.update(overrides)
    return lib.copy_raw(**args), lib.last_error()


@pytest.mark.parametrize(
    "overrides, status, message",
    [
        (dict(key_cache=0), cabi.RK_KV_ERR_INVALID_ARGUMENT, "must not be NULL"),
        (dict(block_mapping=0), cabi.RK_KV_ERR_INVALID_ARGUMENT, "must not be NULL"),
        (dict(dtype=9), cabi.RK_KV_ERR_INVALID_ARGUMENT, "dtype"),
        (dict(index_dtype=-1), cabi.RK_KV_ERR_INVALID_ARGUMENT, "index_dtype"),
        (dict(pairs=0), cabi.RK_KV_ERR_INVALID_ARGUMENT, "positive"),
        (dict(value_cache=72), cabi.RK_KV_ERR_UNSUPPORTED, "16-byte aligned"),
        (dict(block_size=1, kv_heads=1, head_dim=7), cabi.RK_KV_ERR_UNSUPPORTED, "multiple of 16 bytes"),
        (dict(pairs=(1 << 30) + 1), cabi.RK_KV_ERR_UNSUPPORTED, "2^31"),
    ],
)
@cpu_only
def test_kv_copy_invalid_arguments_are_rejected_before_launch(kvlib, overrides, status, message):
    got, text = kv_copy_call(kvlib, **overrides)
    assert got == status, text
    assert message in text


# ---------------------------------------------------------------------------------------------
# Self-attention library (include/rk_sdpa.h).
SDPA_HEADER = ROOT / "include" / "rk_sdpa.h"


@pytest.fixture(scope="module")
def sdpalib():
    if not cabi.SDPA_LIBRARY_PATH.is_file():
        pytest.fail(f"{cabi.SDPA_LIBRARY_PATH} is not built; run __graft_entry__.build()")
    return cabi.SdpaLibrary()


def test_sdpa_header_and_library_agree(sdpalib):
    text = SDPA_HEADER.read_text()
    declared = sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(rk_\w+)\s*\(", text, flags=re.MULTILINE)))
    assert declared == sorted(cabi.SDPA_EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(sdpalib.lib, name), name
    for name in ("RK_SDPA_OK", "RK_SDPA_ERR_INVALID_ARGUMENT", "RK_SDPA_ERR_UNSUPPORTED", "RK_SDPA_ERR_LAUNCH"):
        assert getattr(cabi, name) == int(re.search(rf"#define {name} (\d+)", text).group(1)), name
    assert int(re.search(r"#define RK_SDPA_DTYPE_BF16 (\d+)", text).group(1)) == cabi.RK_DTYPE_BF16
    assert sdpalib.version() == "rk_sdpa_gfx950 1.0.0 (gfx950, wave64)"


@cpu_only
@pytest.mark.parametrize("overrides, status, message", [
    (dict(query=0), cabi.RK_SDPA_ERR_INVALID_ARGUMENT, "must not be NULL"),
    (dict(dtype=3), cabi.RK_SDPA_ERR_INVALID_ARGUMENT, "dtype"),
    (dict(sequence=0), cabi.RK_SDPA_ERR_INVALID_ARGUMENT, "positive"),
    (dict(head_dim=96), cabi.RK_SDPA_ERR_INVALID_ARGUMENT, "one of 64, 128, 256"),
    (dict(query_heads=12, kv_heads=8), cabi.RK_SDPA_ERR_INVALID_ARGUMENT, "divisible"),
    (dict(is_causal=2), cabi.RK_SDPA_ERR_INVALID_ARGUMENT, "is_causal"),
    (dict(scale=float("nan")), cabi.RK_SDPA_ERR_INVALID_ARGUMENT, "positive and finite"),
    (dict(output=104), cabi.RK_SDPA_ERR_UNSUPPORTED, "16-byte aligned"),
    (dict(sequence=1 << 30), cabi.RK_SDPA_ERR_UNSUPPORTED, "launch limits"),
    # 2^24 (sequence, head) rows of 128 query blocks: 2^31 workgroups, too many for either grid order.
    (dict(batch=4096, query_heads=4096, kv_heads=4096, sequence=16384), cabi.RK_SDPA_ERR_UNSUPPORTED,
     "launch limits"),
])
def test_sdpa_invalid_arguments_are_rejected_before_launch(sdpalib, overrides, status, message):
    args = dict(query=16, key=32, value=48, output=96, batch=1, query_heads=8, kv_heads=2, sequence=64,
                head_dim=128, is_causal=1, scale=0.125, dtype=cabi.RK_DTYPE_BF16, stream=0)
    args.update(overrides)
    assert sdpalib.forward_raw(**args) == status
    assert message in sdpalib.last_error()


@cpu_only
@pytest.mark.parametrize("batch, query_heads, kv_heads, sequence, head_dim", [
    (1024, 64, 8, 64, 128),      # 65536 (sequence, head) rows: past the 2-D grid, fine for the 1-D one
    (1, 65536, 65536, 128, 64),
    (1024, 256, 256, 1 << 19, 256),  # the corner of the broad dispatch region
])
def test_sdpa_grids_past_the_two_dimensional_limits_are_launched(sdpalib, batch, query_heads, kv_heads, sequence,
                                                                 head_dim):
    """Grids of several rounds take the one-dimensional XCD-owned order, which has no 65536 limit on
    (sequence x head) rows or query blocks: validation accepts them, and without a GPU the launch
    itself is what fails."""

    got = sdpalib.forward_raw(query=16, key=32, value=48, output=96, batch=batch, query_heads=query_heads,
                              kv_heads=kv_heads, sequence=sequence, head_dim=head_dim, is_causal=1, scale=0.125,
                              dtype=cabi.RK_DTYPE_BF16, stream=0)
    assert got == cabi.RK_SDPA_ERR_LAUNCH, sdpalib.last_error()
    assert "sdpa launch failed" in sdpalib.last_error()
