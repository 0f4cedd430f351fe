"""The C-ABI boundary without a GPU.

Loads ``libfa_gfx950.so`` (loading needs no device), checks that it exports
every entry point ``include/fa_gfx950.h`` declares, that the ctypes binding
passes as many arguments as each declaration takes, and exercises the
host-only paths: ``fa_version``, ``fa_fwd_kvcache_plan`` and the argument
validation every compute entry point runs before touching the device.
Also checks that the Python API rejects bad arguments with the reference's
exception types before any kernel launch.
"""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from flash_attn_triton import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "fa_gfx950.h"


def _declarations():
    """name -> number of parameters, from the header's prototypes."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"^(?:int|const char\*)\s+(fa_\w+)\(([^)]*)\);", text, flags=re.M):
        params = m.group(2).strip()
        decls[m.group(1)] = 0 if params in ("", "void") else len(params.split(","))
    return decls


@pytest.fixture(scope="module")
def lib():
    return _native.load()


def test_header_declares_the_entry_points():
    decls = _declarations()
    for name in ("fa_version", "fa_last_error_string", "fa_fwd_dense", "fa_fwd_varlen",
                 "fa_fwd_kvcache_plan", "fa_fwd_kvcache", "fa_attn_probs", "fa_quant_k_int8",
                 "fa_fwd_int8"):
        assert name in decls, name


def test_library_exports_every_declared_symbol(lib):
    for name in _declarations():
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"


def test_ctypes_binding_matches_header_arity():
    decls = _declarations()
    assert set(_native._SIGNATURES) == set(decls)
    for name, (_, args) in _native._SIGNATURES.items():
        assert len(args) == decls[name], f"{name}: binding {len(args)} vs header {decls[name]}"


def test_version(lib):
    assert lib.fa_version() >= 100


def _plan(lib, *args):
    splits = ctypes.c_int32(-1)
    ws = ctypes.c_int64(-1)
    status = lib.fa_fwd_kvcache_plan(*args, ctypes.byref(splits), ctypes.byref(ws))
    return status, splits.value, ws.value


def test_kvcache_plan_host_only(lib):
    # Decode-shaped (one query row per sequence): split-KV with a workspace
    # that holds fp32 partial outputs and LSEs for every split.
    status, splits, ws = _plan(lib, 4, 1, 32, 8, 128, 8192, 0)
    assert status == _native.FA_OK
    assert splits >= 1
    assert ws >= splits * 4 * 32 * 128 * 4
    # Short caches need no split and no workspace.
    status, splits, ws = _plan(lib, 1, 1, 8, 8, 64, 16, 0)
    assert status == _native.FA_OK and splits == 1 and ws == 0


def test_kvcache_plan_rejects_bad_sizes(lib):
    status, _, _ = _plan(lib, 1, 1, 6, 4, 128, 100, 0)     # Hq not a multiple of Hk
    assert status == _native.FA_ERR_INVALID
    assert lib.fa_last_error_string()
    status, _, _ = _plan(lib, 1, 1, 8, 8, 48, 100, 0)      # unsupported head dim
    assert status == _native.FA_ERR_UNSUPPORTED


def test_entry_points_reject_null_pointers_without_a_device(lib):
    st = _native._strides((0, 0, 0))
    status = lib.fa_fwd_dense(None, None, None, None, None, 1, 1, 1, 1, 1, 64, st, st, st, st,
                              None, 0, 1.0, 0, 0, -1, -1, 0.0, None, 0, None, None, 0.0, 0, None)
    assert status == _native.FA_ERR_INVALID
    assert b"null pointer" in lib.fa_last_error_string()
    status = lib.fa_attn_probs(None, None, None, None, None, None, None, 1, 1, 1, 1, 1, 64, st,
                               st, st, 0, 1.0, 0, 0, -1, -1, 0.0, None, 0, None, None, 0.0, 0,
                               None)
    assert status == _native.FA_ERR_INVALID


def test_dense_rejects_unsupported_dtype_and_head_dim(lib):
    st = _native._strides((1024, 64, 64))
    one = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    status = lib.fa_fwd_dense(one, one, one, one, None, 1, 1, 1, 1, 1, 64, st, st, st, st,
                              None, 7, 1.0, 0, 0, -1, -1, 0.0, None, 0, None, None, 0.0, 0, None)
    assert status == _native.FA_ERR_UNSUPPORTED
    status = lib.fa_fwd_dense(one, one, one, one, None, 1, 1, 1, 1, 1, 40, st, st, st, st,
                              None, 0, 1.0, 0, 0, -1, -1, 0.0, None, 0, None, None, 0.0, 0, None)
    assert status == _native.FA_ERR_UNSUPPORTED


def test_python_api_validation_on_cpu():
    """Checks the reference runs before any launch (flash_attn_interface.py:96-127)."""
    from flash_attn_triton import flash_attn_func, flash_attn_varlen_func
    q = torch.zeros(1, 4, 2, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="CUDA"):
        flash_attn_func(q, q, q)
    with pytest.raises(ValueError, match="softcap"):
        flash_attn_func(q, q, q, softcap=-1.0)
    with pytest.raises(ValueError, match="dropout_p"):
        flash_attn_func(q, q, q, dropout_p=1.0)
    with pytest.raises(ValueError):
        flash_attn_func(q.to(torch.int32), q, q)
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(ValueError):
        flash_attn_varlen_func(q[0], q[0], q[0], cu, torch.tensor([0, 2, 4], dtype=torch.int32),
                               4, 4)


def test_deferred_checks_keep_the_reference_order():
    """Device-side checks are read with one synchronization, but a later host
    check never overtakes an earlier failing device check."""
    from flash_attn_triton._checks import Deferred
    chk = Deferred()
    chk.check(torch.tensor(False), ValueError("first"))
    chk.check(torch.tensor(True), ValueError("second"))
    with pytest.raises(ValueError, match="second"):
        chk.fail(RuntimeError("host"))
    chk = Deferred()
    chk.check(torch.tensor(False), ValueError("first"))
    with pytest.raises(RuntimeError, match="host"):
        chk.fail(RuntimeError("host"))
    chk = Deferred()
    i = chk.value(torch.tensor(7))
    chk.check(torch.tensor(False), ValueError("never"))
    assert chk.flush()[i] == 7
    assert chk.flush() == []


def test_varlen_cu_seqlens_errors_before_device_errors():
    """Reference order (flash_attn_interface.py:583-598): cu_seqlens checks run
    before the CUDA-tensor check."""
    from flash_attn_triton import flash_attn_varlen_func
    q = torch.zeros(4, 2, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="start at zero"):
        flash_attn_varlen_func(q, q, q, torch.tensor([1, 4], dtype=torch.int32),
                               torch.tensor([0, 4], dtype=torch.int32), 4, 4)
    with pytest.raises(ValueError, match="monotonically"):
        flash_attn_varlen_func(q, q, q, torch.tensor([0, 3, 2, 4], dtype=torch.int32),
                               torch.tensor([0, 1, 2, 4], dtype=torch.int32), 4, 4)
    with pytest.raises(ValueError, match="exceed"):
        flash_attn_varlen_func(q, q, q, torch.tensor([0, 5], dtype=torch.int32),
                               torch.tensor([0, 4], dtype=torch.int32), 4, 4)
    with pytest.raises(ValueError, match="CUDA tensors"):
        flash_attn_varlen_func(q, q, q, torch.tensor([0, 4], dtype=torch.int32),
                               torch.tensor([0, 4], dtype=torch.int32), 4, 4)


def test_noalloc_rejects_workspace_beyond_scratch_without_a_device(lib):
    # The no-allocation KV-cache entry point checks the split workspace its
    # plan needs against the fixed scratch array before touching any device.
    st = _native._strides((4096, 4096, 128))
    one = ctypes.c_void_p(16)   # never dereferenced: the size check fails first
    args = (one, one, one, one, None, one, one, 32, 256, 64, None, None,
            4096, 1, 8192, 32, 8, 128, st, st, st, st, None, 0, 0.088, 0, -1, -1, None, 0, None)
    splits, ws = _native.kvcache_plan(4096, 1, 32, 8, 128, 8192, 256)
    assert ws > (16 << 20)
    status = lib.fa_fwd_kvcache_noalloc(*args)
    assert status == _native.FA_ERR_UNSUPPORTED
    assert b"scratch" in lib.fa_last_error_string()


def _integration_snippet():
    """The reference-side binding that INTEGRATION.md shows a maintainer (the
    first Python block that loads the library), executed with its ``CDLL``
    pointed at this build's library (a fresh handle, so the snippet's argtypes
    do not touch the package's own binding)."""
    text = (Path(__file__).resolve().parents[1] / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    code = next(b for b in blocks if "ctypes.CDLL" in b)
    real_cdll = ctypes.CDLL
    ns = {}
    try:
        ctypes.CDLL = lambda name, *a, **kw: real_cdll(str(_native.library_path()), *a, **kw)
        exec(compile(code, "INTEGRATION.md", "exec"), ns)
    finally:
        ctypes.CDLL = real_cdll
    return ns


def test_integration_binding_matches_header_and_dtype_codes():
    """The documented ctypes stub passes fa_fwd_dense's arguments with the
    header's arity and the package's argument types, and maps dtypes to the
    header's FA_DTYPE_* codes: fp16 -> FA_DTYPE_F16, fp32 -> FA_DTYPE_F32;
    anything the reference rejects (flash_attn_interface.py:95-96) raises."""
    ns = _integration_snippet()
    args = ns["_lib"].fa_fwd_dense.argtypes
    assert len(args) == _declarations()["fa_fwd_dense"]
    assert list(args) == list(_native._SIGNATURES["fa_fwd_dense"][1])
    codes = dict(re.findall(r"#define (FA_DTYPE_\w+) (\d+)", HEADER.read_text()))
    assert ns["_dtype_code"](torch.float16) == int(codes["FA_DTYPE_F16"]) \
        == _native.dtype_code(torch.float16)
    assert ns["_dtype_code"](torch.float32) == int(codes["FA_DTYPE_F32"]) \
        == _native.dtype_code(torch.float32)
    for bad in (torch.bfloat16, torch.float64, torch.int32):
        with pytest.raises(ValueError):
            ns["_dtype_code"](bad)


def test_kvcache_empty_batch_needs_no_workspace(lib):
    # batch == 0 launches nothing, so the NULL workspace the header allows
    # for a size-0 plan is accepted even where the plan would split; the
    # no-allocation variant returns before touching its scratch array.
    st = _native._strides((4096, 4096, 128))
    one = ctypes.c_void_p(16)   # never dereferenced: nothing is launched
    head = (one, one, one, one, None, one, one, 32, 256, 64, None, None)
    tail = (st, st, st, st, None, _native.FA_DTYPE_F16, 0.088, 0, -1, -1, None, 0)
    splits, _ = _native.kvcache_plan(0, 1, 32, 8, 128, 8192, 256)
    assert lib.fa_fwd_kvcache(*head, 0, 1, 8192, 32, 8, 128, *tail, splits, None, 0,
                              None) == _native.FA_OK
    assert lib.fa_fwd_kvcache_noalloc(*head, 0, 1, 8192, 32, 8, 128, *tail,
                                      None) == _native.FA_OK

