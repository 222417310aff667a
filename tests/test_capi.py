"""The C-ABI library loads on a host without a GPU and exports every entry point the
header declares; argument checks reject bad calls before any device work."""
import ctypes
import pathlib
import re

import pytest

from polyhedral_amd import _lib

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "polyattn_amd.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(pa_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = _declared()
    assert "pa_attn_fwd" in names and "pa_index_classify" in names
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures and the header disagree"


def test_abi_version_and_error_channel():
    lib = _lib.lib()
    assert lib.pa_abi_version() == _lib.ABI_VERSION
    m = _lib.PaMask()
    m.n_include = 1
    rc = lib.pa_index_classify(ctypes.byref(m), 1000, 48, 32, None, None, None, None)
    assert rc == _lib.PA_E_INVALID
    assert b"null argument" in lib.pa_last_error() or b"BQ" in lib.pa_last_error()
    buf = (ctypes.c_int32 * 4)()
    rc = lib.pa_index_classify(ctypes.byref(m), 1000, 48, 32, buf, buf, buf, None)
    assert rc == _lib.PA_E_INVALID and b"BQ=48" in lib.pa_last_error()


def test_attention_argument_checks_run_before_any_launch():
    lib = _lib.lib()
    a = _lib.PaAttnArgs()
    assert lib.pa_attn_fwd(ctypes.byref(a), None) == _lib.PA_E_INVALID      # null tensors
    buf = (ctypes.c_int64 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    a.q = a.k = a.v = a.o = a.kv_idx = a.kv_num = a.kv_partial = p
    a.D, a.dtype, a.BH, a.N, a.BQ, a.A = 96, _lib.PA_BF16, 1, 1024, 128, 32
    assert lib.pa_attn_fwd(ctypes.byref(a), None) == _lib.PA_E_INVALID
    assert b"D=96" in lib.pa_last_error()
    a.D, a.N = 128, 1000
    assert lib.pa_attn_fwd(ctypes.byref(a), None) == _lib.PA_E_INVALID
    assert b"not divisible" in lib.pa_last_error()
    a.N, a.mask.n_include = 1024, 0
    assert lib.pa_attn_fwd(ctypes.byref(a), None) == _lib.PA_E_INVALID
    assert b"n_include" in lib.pa_last_error()


def test_struct_layouts_match_the_header():
    """ctypes field offsets of pa_attn_args follow the C layout (spot checks)."""
    off = {f[0]: getattr(_lib.PaAttnArgs, f[0]).offset for f in _lib.PaAttnArgs._fields_}
    assert off["q"] == 0 and off["q_sb"] == 32 and off["BH"] == 96 and off["D"] == 112
    assert off["kv_idx"] % 8 == 0 and off["mask"] % 8 == 0
    assert ctypes.sizeof(_lib.PaMask) == 8 + 16 * _lib.MAX_TERMS + 8 * 4


def test_product_refuses_host_tensors():
    """No host fallback: the drop-in entry points raise on CPU tensors."""
    import torch

    from polyhedral_amd import attention, perm
    q = torch.zeros(1, 128, 64)
    idx = torch.zeros(1, 1, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU only"):
        attention.block_sparse_attention(q, q, q, idx, torch.ones(1, dtype=torch.int32),
                                         torch.zeros(1, 1, dtype=torch.int8), 0, 0, 0, 0, 128, 128)
    with pytest.raises(RuntimeError, match="GPU only"):
        perm.apply_perm(q, torch.arange(128, dtype=torch.int32))


def test_every_struct_field_offset_matches_the_c_compiler(tmp_path):
    """gcc compiles the header and prints offsetof / sizeof of every field of pa_attn_args,
    pa_mask, pa_term, pa_decode_args, pa_attn_bwd_args and pa_split_args; the ctypes mirrors must agree
    field by field."""
    import shutil
    import subprocess
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    structs = {"pa_attn_args": _lib.PaAttnArgs, "pa_mask": _lib.PaMask, "pa_term": _lib.PaTerm,
               "pa_decode_args": _lib.PaDecodeArgs, "pa_attn_bwd_args": _lib.PaAttnBwdArgs,
               "pa_split_args": _lib.PaSplitArgs}
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'  printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'  printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("  return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-o", str(exe), str(src)], check=True, capture_output=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    seen = 0
    for line in filter(None, out):
        cname, field, val = line.split()
        cls = structs[cname]
        want = ctypes.sizeof(cls) if field == "sizeof" else getattr(cls, field).offset
        assert int(val) == want, f"{cname}.{field}: C {val}, ctypes {want}"
        seen += 1
    assert seen == sum(len(c._fields_) + 1 for c in structs.values())


def test_backward_argument_checks_run_before_any_launch():
    lib = _lib.lib()
    a = _lib.PaAttnBwdArgs()
    assert lib.pa_attn_bwd(ctypes.byref(a), None) == _lib.PA_E_INVALID      # dtype 0 (fp32)
    buf = (ctypes.c_int64 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    for f in ("q", "k", "v", "o", "dout", "dq", "dk", "dv", "lse", "dvec", "kv_idx", "kv_num", "kv_partial",
              "q_idx", "q_num", "q_partial"):
        setattr(a, f, p)
    a.dtype, a.D, a.BH, a.N, a.sb, a.sn, a.pitch, a.tpitch = _lib.PA_BF16, 128, 2, 1024, 1024 * 128, 128, 4, 4
    a.lse_sb = 1024
    a.mask.n_include = 1
    a.kv_bits = p                                                           # one of four bitmap arrays
    assert lib.pa_attn_bwd(ctypes.byref(a), None) == _lib.PA_E_INVALID
    assert b"bitmap" in lib.pa_last_error()
    a.kv_bits = None
    a.flags = 4
    assert lib.pa_attn_bwd(ctypes.byref(a), None) == _lib.PA_E_INVALID
    assert b"flags" in lib.pa_last_error()
    a.flags, a.residue_s = 1, 24                                            # 1024 / 24 is not whole
    assert lib.pa_attn_bwd(ctypes.byref(a), None) == _lib.PA_E_INVALID
    assert b"residue_s=24" in lib.pa_last_error()
    a.residue_s, a.D = 16, 64                                               # residue basis needs D = 128
    assert lib.pa_attn_bwd(ctypes.byref(a), None) == _lib.PA_E_INVALID
    assert b"residue_s=16" in lib.pa_last_error()
    a.residue_s, a.N = 0, 1000
    assert lib.pa_attn_bwd(ctypes.byref(a), None) == _lib.PA_E_INVALID
    assert b"multiple of 64" in lib.pa_last_error()
    # the transpose entry points
    assert lib.pa_index_transpose(p, p, p, None, 0, 4, 16, p, None, None, None, 0, None) == _lib.PA_E_INVALID
    assert lib.pa_index_transpose(p, p, None, None, 16, 4, 16, p, None, None, None, 0, None) == _lib.PA_E_INVALID
    assert b"kv_partial" in lib.pa_last_error()
    assert lib.pa_index_transpose(p, p, p, None, 16, 4, 16, p, p, p, p, 4, None) == _lib.PA_E_INVALID
    assert b"q_bits_off" in lib.pa_last_error()
    assert lib.pa_index_bits_transpose(None, 16, 4, p, p, None) == _lib.PA_E_INVALID
    assert lib.pa_index_bits_transpose(p, 16, 0, None, None, None) == _lib.PA_OK   # nothing listed


def test_backward_rejects_lse_rows_shorter_than_n():
    """lse and dvec rows of stride lse_sb < N would overlap (an expanded lse has stride 0)."""
    lib = _lib.lib()
    a = _lib.PaAttnBwdArgs()
    buf = (ctypes.c_int64 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    for f in ("q", "k", "v", "o", "dout", "dq", "dk", "dv", "lse", "dvec", "kv_idx", "kv_num", "kv_partial",
              "q_idx", "q_num", "q_partial"):
        setattr(a, f, p)
    a.dtype, a.D, a.BH, a.N, a.sb, a.sn, a.pitch, a.tpitch = _lib.PA_BF16, 128, 2, 1024, 1024 * 128, 128, 4, 4
    a.mask.n_include = 1
    for sb in (0, 512, 1023):
        a.lse_sb = sb
        assert lib.pa_attn_bwd(ctypes.byref(a), None) == _lib.PA_E_INVALID
        assert b"lse_sb" in lib.pa_last_error()


def test_backward_host_checks_on_lse_layout():
    """The Python layer gives dvec lse's strides and refuses an lse whose rows overlap."""
    import torch

    from polyhedral_amd import backward as pbwd
    plan = pbwd.BackwardPlan.__new__(pbwd.BackwardPlan)
    plan.N = 64
    q = torch.zeros(2, 64, 128, dtype=torch.bfloat16)
    for lse in (torch.zeros(1, 64).expand(2, 64),     # row stride 0
                torch.zeros(2, 32)):                  # rows shorter than N
        with pytest.raises(ValueError, match="lse must be"):
            plan.backward(q, q, q, q, lse, q)


@pytest.mark.parametrize("BH,cap,length,s,splits", [
    (32, 16384, 16384, 16, 16),   # 4 groups per class, 16 classes: 16 work-groups per head
    (32, 16384, 16384, 0, 16),    # identity: 64 groups, 512 / 32 work-groups per head
    (1, 16384, 16384, 0, 64),     # one head: a work-group per group
    (8, 65536, 65536, 32, 64),
    (64, 4096, 4000, 16, 8),
    (3, 1024, 1, 16, 16),         # one entry: every class is one (mostly empty) group
    (2, 2048, 0, 8, 0),           # empty cache: no split launch
    (65535, 256, 256, 0, 1),
])
def test_decode_split_plan(BH, cap, length, s, splits):
    """The decode split plan, read back through pa_decode_workspace (BH * splits * nq *
    (D + 1) floats): about 512 work-groups in all, never more per head than there are
    256-entry groups, none for an empty cache."""
    lib = _lib.lib()
    a = _lib.PaDecodeArgs()
    buf = (ctypes.c_int64 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    a.q, a.k_cache, a.v_cache, a.o = p, p, p, p
    a.nq, a.BH, a.D, a.dtype = 1, BH, 128, _lib.PA_BF16
    a.q_sb, a.q_sn, a.c_sb, a.c_sn, a.o_sb, a.o_sn = 128, 128, cap * 128, 128, 128, 128
    a.capacity, a.length, a.residue_s = cap, length, s
    a.mask.n_include = 1
    n = ctypes.c_int64(-1)
    assert lib.pa_decode_workspace(ctypes.byref(a), ctypes.byref(n)) == _lib.PA_OK
    assert n.value % (BH * 129 * 4) == 0
    got = n.value // (BH * 129 * 4)
    assert got == splits
    classes = max(s, 1)
    groups = classes * -(-(-(-length // classes)) // 256)   # 256-entry groups of the head
    assert got <= min(512, groups)


def test_decode_rejects_residue_bases_beyond_4096_classes():
    """A cache's basis has at most 4096 classes (an earlier split planner had no exit past
    that); a larger residue_s is an argument error."""
    lib = _lib.lib()
    a = _lib.PaDecodeArgs()
    buf = (ctypes.c_int64 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    a.q, a.k_cache, a.v_cache, a.o = p, p, p, p
    a.nq, a.BH, a.D, a.dtype = 1, 1, 128, _lib.PA_BF16
    a.q_sb, a.q_sn, a.c_sb, a.c_sn, a.o_sb, a.o_sn = 128, 128, 16384 * 128, 128, 128, 128
    a.capacity, a.length, a.residue_s = 16384, 100, 8192
    a.mask.n_include = 1
    n = ctypes.c_int64(0)
    assert lib.pa_decode_workspace(ctypes.byref(a), ctypes.byref(n)) == _lib.PA_E_INVALID
    assert b"residue_s=8192" in lib.pa_last_error()
    assert lib.pa_kv_append(p, p, 128, 128, p, p, 16384 * 128, 128, 1, 1, 128, _lib.PA_BF16, 16384, 0, 8192,
                            None) == _lib.PA_E_INVALID
    assert b"residue_s=8192" in lib.pa_last_error()
    a.residue_s = 4096                                 # the largest accepted basis plans normally
    assert lib.pa_decode_workspace(ctypes.byref(a), ctypes.byref(n)) == _lib.PA_OK and n.value > 0
    from polyhedral_amd import decode as pdec
    with pytest.raises(ValueError):
        pdec.KVCache(1, 16384, 128, residue=8192, device="cpu")


def test_decode_append_arguments_are_checked():
    """The tokens a decode call appends (n_new > 0) must be at most 8, inside the attended
    length, with both row pointers given and 16-byte aligned; the host checks refuse
    them before touching a device."""
    lib = _lib.lib()
    a = _lib.PaDecodeArgs()
    buf = (ctypes.c_int64 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    a.q, a.k_cache, a.v_cache, a.o = p, p, p, p
    a.nq, a.BH, a.D, a.dtype = 1, 2, 128, _lib.PA_BF16
    a.q_sb, a.q_sn, a.c_sb, a.c_sn, a.o_sb, a.o_sn = 128, 128, 1024 * 128, 128, 128, 128
    a.capacity, a.length, a.residue_s = 1024, 100, 16
    a.mask.n_include = 1
    n = ctypes.c_int64(0)
    assert lib.pa_decode_workspace(ctypes.byref(a), ctypes.byref(n)) == _lib.PA_OK
    a.n_new, a.new_pos0, a.new_sb, a.new_sn = 1, 99, 128, 128
    assert lib.pa_decode_workspace(ctypes.byref(a), ctypes.byref(n)) == _lib.PA_E_INVALID
    assert b"k_new" in lib.pa_last_error()
    a.k_new, a.v_new = p, p
    assert lib.pa_decode_workspace(ctypes.byref(a), ctypes.byref(n)) == _lib.PA_OK
    for field, value, text in (("n_new", 9, b"n_new=9"), ("new_pos0", 100, b"outside the attended length"),
                               ("new_sn", 100, b"16-byte aligned")):
        old = getattr(a, field)
        setattr(a, field, value)
        assert lib.pa_decode_workspace(ctypes.byref(a), ctypes.byref(n)) == _lib.PA_E_INVALID, field
        assert text in lib.pa_last_error(), (field, lib.pa_last_error())
        setattr(a, field, old)


def test_static_decode_rejects_a_workspace_and_partials_beyond_its_scratch():
    """pa_decode_fwd_static takes no workspace, and refuses (before touching a device) a
    call whose split partials exceed its 8 MiB scratch."""
    lib = _lib.lib()
    a = _lib.PaDecodeArgs()
    buf = (ctypes.c_int64 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    a.q, a.k_cache, a.v_cache, a.o = p, p, p, p
    a.nq, a.BH, a.D, a.dtype = 8, 4096, 128, _lib.PA_BF16
    a.q_sb, a.q_sn, a.c_sb, a.c_sn, a.o_sb, a.o_sn = 1024, 128, 256 * 128, 128, 1024, 128
    a.capacity, a.length, a.residue_s = 256, 256, 0
    a.mask.n_include = 1
    n = ctypes.c_int64(0)
    assert lib.pa_decode_workspace(ctypes.byref(a), ctypes.byref(n)) == _lib.PA_OK
    assert n.value == 4096 * 8 * 129 * 4 > 8 << 20
    assert lib.pa_decode_fwd_static(ctypes.byref(a), None) == _lib.PA_E_INVALID
    assert b"scratch" in lib.pa_last_error()
    a.BH = 1
    a.workspace, a.workspace_bytes = p, 512
    assert lib.pa_decode_fwd_static(ctypes.byref(a), None) == _lib.PA_E_INVALID
    assert b"takes no workspace" in lib.pa_last_error()
