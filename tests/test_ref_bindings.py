"""The reference's Python seam (scripts/kcmm/bindings.py, the loader its
vLLM patches use) against this library: every C entry point it declares is
exported, with the argument and return ABI kinds it declares equal to this
build's signatures (lattice_amd/bindings.py, which mirror include/kcmm.h).
The reference's declarations are a committed fixture
(tests/golden/ref_bindings_signatures.json, written by
tests/golden/make_ref_bindings.py from the file's text)."""
import ctypes as C
import json
from pathlib import Path

import pytest

from lattice_amd.bindings import SIGNATURES

FIXTURE = Path(__file__).parent / "golden" / "ref_bindings_signatures.json"


def kind(t):
    if t is None:
        return "void"
    if t in (C.c_void_p, C.c_char_p) or isinstance(t, type(C.POINTER(C.c_int))):
        return "ptr"
    return {C.c_uint32: "u32", C.c_uint64: "u64", C.c_size_t: "u64", C.c_int: "i32",
            C.c_int32: "i32", C.c_float: "f32", C.c_int64: "i64"}[t]


REF = json.loads(FIXTURE.read_text())["functions"]


@pytest.mark.parametrize("name", sorted(REF))
def test_reference_seam_entry_point(hostcheck_lib, name):
    assert hasattr(hostcheck_lib.lib, name), f"{name} not exported"
    ref = REF[name]
    ours_args, ours_ret = SIGNATURES[name]
    norm = lambda k: "u64" if k == "size" else k   # size_t is 64-bit on this ABI
    if "args" in ref:
        assert [norm(k) for k in ref["args"]] == [kind(t) for t in ours_args], name
    if "ret" in ref:
        assert norm(ref["ret"]) == kind(ours_ret), name


def test_fixture_covers_the_seam():
    # the reference seam's core: pool lifecycle, allocation, tables, KV write
    # by slot, attention
    for name in ("kcmm_pool_create", "kcmm_alloc_blocks", "kcmm_append_kv_slots_on_stream",
                 "kcmm_paged_attn_decode_f16_on_stream", "kcmm_get_all_block_offsets_f16"):
        assert name in REF
