"""The C-ABI libraries: they load on a machine without a GPU and export every function
their header declares (include/fdllm_hip.h: libfdllm_hip.so, whose ctypes table binds
exactly those functions; include/fdllm_probes.h: libfdllm_probes.so, the measurement
probes bench.py uses). No kernel is launched here; argument checks that reject a call
before any launch are exercised through the C ABI with null pointers.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADERS = [ROOT / "include" / "fdllm_hip.h"]
PROBES_HEADER = ROOT / "include" / "fdllm_probes.h"
PROBES_LIB = ROOT / "fast_v2_amd" / "lib" / "libfdllm_probes.so"


def test_every_header_is_checked():
    assert sorted((ROOT / "include").glob("*.h")) == sorted(HEADERS + [PROBES_HEADER])


def _declared_functions(headers=HEADERS):
    names = set()
    for h in headers:
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b(fdllm_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def lib():
    from fast_v2_amd import _ffi
    if not _ffi.LIB_PATH.exists():
        pytest.fail(f"{_ffi.LIB_PATH} is not built (run __graft_entry__.build())")
    return _ffi.lib()


def test_header_declares_the_entry_points():
    names = _declared_functions()
    assert {"fdllm_gather_rmsnorm", "fdllm_scatter_rows", "fdllm_kv_attn_fwd",
            "fdllm_kv_attn_workspace_size", "fdllm_kv_cache_write", "fdllm_rope_kv_write", "fdllm_abi_version",
            "fdllm_last_error"} <= names


def test_library_exports_every_declared_symbol(lib):
    from fast_v2_amd import _ffi
    out = subprocess.run(["nm", "-D", "--defined-only", str(_ffi.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = _declared_functions() - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"
    for name in _declared_functions():
        assert getattr(lib, name) is not None


def test_probes_library_exports_its_header():
    if not PROBES_LIB.exists():
        pytest.fail(f"{PROBES_LIB} is not built (run __graft_entry__.build())")
    names = _declared_functions([PROBES_HEADER])
    assert names == {"fdllm_probe_read_kv", "fdllm_probe_copy_rows", "fdllm_probe_mfma"}
    out = subprocess.run(["nm", "-D", "--defined-only", str(PROBES_LIB)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert names <= exported
    lib = ctypes.CDLL(str(PROBES_LIB))
    # rejected arguments return before any launch (no GPU needed)
    lib.fdllm_probe_copy_rows.restype = ctypes.c_int
    assert lib.fdllm_probe_copy_rows(None, 16, 1, None, None, 1, 16, None) == -1
    lib.fdllm_probe_read_kv.restype = ctypes.c_int
    assert lib.fdllm_probe_read_kv(*([None] * 2 + [0] * 6 + [None, 0, 32, None, 1, 4, 64, None, None])) == -1
    lib.fdllm_probe_mfma.restype = ctypes.c_int
    assert lib.fdllm_probe_mfma(256, 8, None, None) == -1


def test_ctypes_table_matches_header():
    from fast_v2_amd import _ffi
    assert set(_ffi.SIGNATURES) == _declared_functions()


def test_abi_version_and_error_string(lib):
    assert lib.fdllm_abi_version() == 2
    assert isinstance(lib.fdllm_last_error(), bytes)


def test_descriptor_layout_matches_c_struct():
    """ctypes mirror of fdllm_kv_attn_desc: field order and offsets follow C layout rules."""
    from fast_v2_amd import _ffi
    d = _ffi.KVAttnDesc
    assert d.q.offset == 0
    assert d.k.offset == 32 and d.v.offset == 64 and d.out.offset == 96
    assert d.page_table.offset == 128 and d.seqlens.offset == 136 and d.q_start.offset == 144
    assert d.max_pages.offset == 152
    assert d.softmax_scale.offset == d.kv_split.offset + 4
    assert ctypes.sizeof(d) % 8 == 0


@pytest.mark.parametrize("struct", ["fdllm_kv_attn_desc", "fdllm_rope_kv_desc", "fdllm_qkv_rope_desc"])
def test_descriptor_offsets_match_the_c_compiler(tmp_path, struct):
    """Every field offset and the size of the ctypes mirrors equal what gcc lays out
    for the structs of include/fdllm_hip.h."""
    from fast_v2_amd import _ffi
    mirror = {"fdllm_kv_attn_desc": _ffi.KVAttnDesc, "fdllm_rope_kv_desc": _ffi.RopeKVDesc,
              "fdllm_qkv_rope_desc": _ffi.QkvRopeDesc}[struct]
    fields = [f[0] for f in mirror._fields_]
    prog = tmp_path / "layout.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{ROOT / "include" / "fdllm_hip.h"}"',
             'int main(void) {', f'  printf("size %zu\\n", sizeof({struct}));']
    lines += [f'  printf("{n} %zu\\n", offsetof({struct}, {n}));' for n in fields]
    lines += ['  return 0;', '}']
    prog.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-o", str(exe), str(prog)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                        check=True).stdout.splitlines())
    assert int(got["size"]) == ctypes.sizeof(mirror)
    for n in fields:
        assert int(got[n]) == getattr(mirror, n).offset, n


def test_rejected_arguments_launch_nothing(lib):
    """Calls that fail validation return a negative code and set the error text."""
    from fast_v2_amd import _ffi
    d = _ffi.KVAttnDesc()
    d.dtype = 99  # no such dtype
    d.head_dim, d.num_q_heads, d.num_kv_heads = 128, 28, 4
    size = ctypes.c_size_t(0)
    rc = lib.fdllm_kv_attn_workspace_size(ctypes.byref(d), ctypes.byref(size))
    assert rc == _ffi.FDLLM_ERR_INVALID_ARGUMENT
    assert b"dtype" in lib.fdllm_last_error()
    d.dtype = _ffi.DTYPE_BF16
    d.num_q_heads = 30  # not a multiple of 4
    assert lib.fdllm_kv_attn_workspace_size(ctypes.byref(d), ctypes.byref(size)) == _ffi.FDLLM_ERR_INVALID_ARGUMENT
    d.num_q_heads = 28
    d.page_table = 16  # any non-null pointer: page size 48 is rejected before use
    d.page_size, d.max_pages = 48, 4
    assert lib.fdllm_kv_attn_workspace_size(ctypes.byref(d), ctypes.byref(size)) == _ffi.FDLLM_ERR_INVALID_ARGUMENT
    assert b"page_size" in lib.fdllm_last_error()
    # a weighted norm mode without a weight is rejected (NULL weight only with NORM_PLAIN)
    rc = lib.fdllm_gather_rmsnorm(None, 0, 0, None, 0, None, 0, None, None, 1, 1, 1, 64, 1e-6,
                                  _ffi.DTYPE_BF16, _ffi.NORM_WEIGHT_AFTER_CAST, None)
    assert rc == _ffi.FDLLM_ERR_INVALID_ARGUMENT
    rc = lib.fdllm_kv_cache_write(None, None, 0, 0, 0, None, None, 0, 0, 0, None, 0, 0, 0, None, 0, None,
                                  1, 1, 4, 128, _ffi.DTYPE_F32, None)
    assert rc == _ffi.FDLLM_ERR_INVALID_ARGUMENT
    r = _ffi.RopeKVDesc()
    r.batch, r.seq_len, r.num_q_heads, r.num_kv_heads, r.head_dim = 1, 1, 28, 4, 128
    r.dtype = _ffi.DTYPE_F32
    assert lib.fdllm_rope_kv_write(ctypes.byref(r), None) == _ffi.FDLLM_ERR_INVALID_ARGUMENT
    assert b"dtype" in lib.fdllm_last_error()
    r.dtype, r.head_dim = _ffi.DTYPE_BF16, 72  # not a multiple of 16
    assert lib.fdllm_rope_kv_write(ctypes.byref(r), None) == _ffi.FDLLM_ERR_INVALID_ARGUMENT
    r.head_dim = 128  # no tensors given
    assert lib.fdllm_rope_kv_write(ctypes.byref(r), None) == _ffi.FDLLM_ERR_INVALID_ARGUMENT
    assert b"null" in lib.fdllm_last_error()
    # fused projections: head_dim other than 128, hidden not a multiple of 64, no tensors
    qd = _ffi.QkvRopeDesc()
    qd.rope.batch, qd.rope.seq_len, qd.rope.num_q_heads, qd.rope.num_kv_heads = 1, 1, 28, 4
    qd.rope.dtype, qd.rope.head_dim, qd.hidden, qd.x_stride_row = _ffi.DTYPE_BF16, 64, 3584, 3584
    assert lib.fdllm_qkv_rope_kv_write(ctypes.byref(qd), None) == _ffi.FDLLM_ERR_INVALID_ARGUMENT
    assert b"head_dim" in lib.fdllm_last_error()
    qd.rope.head_dim, qd.hidden, qd.x_stride_row = 128, 3584 + 32, 3584 + 32
    assert lib.fdllm_qkv_rope_kv_write(ctypes.byref(qd), None) == _ffi.FDLLM_ERR_INVALID_ARGUMENT
    assert b"multiple of 64" in lib.fdllm_last_error()
    qd.hidden, qd.x_stride_row = 3584, 3584
    assert lib.fdllm_qkv_rope_kv_write(ctypes.byref(qd), None) == _ffi.FDLLM_ERR_INVALID_ARGUMENT
    assert b"null" in lib.fdllm_last_error()
    # residual add + norm: hidden size not a multiple of 8; SiLU product: ragged length
    rc = lib.fdllm_add_rmsnorm(None, None, None, 0, None, None, 4, 100, 1e-6, _ffi.DTYPE_BF16, _ffi.NORM_PLAIN, None)
    assert rc == _ffi.FDLLM_ERR_INVALID_ARGUMENT and b"multiple of 8" in lib.fdllm_last_error()
    rc = lib.fdllm_add_rmsnorm(None, None, None, 0, None, None, 4, 64, 1e-6, _ffi.DTYPE_F32, _ffi.NORM_PLAIN, None)
    assert rc == _ffi.FDLLM_ERR_INVALID_ARGUMENT and b"dtype" in lib.fdllm_last_error()
    assert lib.fdllm_silu_mul(None, None, None, 12, _ffi.DTYPE_BF16, None) == _ffi.FDLLM_ERR_INVALID_ARGUMENT
    assert lib.fdllm_silu_mul(None, None, None, 16, _ffi.DTYPE_BF16, None) == _ffi.FDLLM_ERR_INVALID_ARGUMENT
    assert b"null" in lib.fdllm_last_error()


def test_workspace_size_for_the_decode_workload(lib):
    """The bs16 sub-block decode plan is split over several workgroups per sequence and
    asks for a workspace; a tiny single-split call asks for none."""
    from fast_v2_amd import _ffi
    d = _ffi.KVAttnDesc()
    d.dtype = _ffi.DTYPE_BF16
    d.batch, d.q_len, d.num_q_heads, d.num_kv_heads, d.head_dim = 16, 8, 28, 4, 128
    d.k_stride_h = d.v_stride_h = 128
    d.max_seqlen = 4128
    d.softmax_scale = 128 ** -0.5
    size = ctypes.c_size_t(0)
    assert lib.fdllm_kv_attn_workspace_size(ctypes.byref(d), ctypes.byref(size)) == 0
    assert size.value > 0
    d.max_seqlen = 64
    assert lib.fdllm_kv_attn_workspace_size(ctypes.byref(d), ctypes.byref(size)) == 0
    assert size.value == 0


def test_workspace_size_for_the_full_block_workload(lib):
    """The bs16 full-block plan (32 queries x GQA 7 = 224 rows per KV head) splits each
    KV head's keys over 64 slots of 256 rows, one workgroup per compute unit. Its
    workspace holds the 64 KiB of counters, an fp32 (m, l) pair per slot row, one
    (first slot, splits) pair per (sequence, KV head) for the merge kernel (padded to
    256 bytes), and the fp32 partial rows."""
    from fast_v2_amd import _ffi
    d = _ffi.KVAttnDesc()
    d.dtype = _ffi.DTYPE_BF16
    B, Hkv, D = 16, 4, 128
    d.batch, d.q_len, d.num_q_heads, d.num_kv_heads, d.head_dim = B, 32, 28, Hkv, D
    d.k_stride_h = d.v_stride_h = D
    d.max_seqlen = 4128
    d.softmax_scale = D ** -0.5
    size = ctypes.c_size_t(0)
    assert lib.fdllm_kv_attn_workspace_size(ctypes.byref(d), ctypes.byref(size)) == 0
    slot_rows = 64 * Hkv * 256
    ml_and_table = slot_rows * 8 + B * Hkv * 8
    ml_and_table = (ml_and_table + 255) // 256 * 256
    assert size.value == 64 * 1024 + ml_and_table + slot_rows * D * 4
