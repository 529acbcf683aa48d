"""The C-ABI library loads without a GPU and exports every function that
include/*.h declares; the ctypes table and the struct layouts agree with the
headers. No compute call is made here."""
import ctypes
import glob
import os
import re
import subprocess

import pytest

from arclight_amd import _lib, abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))
DECL = re.compile(r"^[A-Za-z_][\w \*]*?\b(al_\w+)\s*\(", re.M)


def declared():
    names = []
    for h in HEADERS:
        names += DECL.findall(open(h).read())
    return sorted(set(names))


def test_headers_declare_functions():
    names = declared()
    assert "al_fattn_f16" in names and "al_set_rows_f32_f16" in names
    assert len(names) >= 30


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built (run python -m arclight_amd.build)")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_ctypes_table_matches_headers():
    assert sorted(_lib.SIGNATURES) == declared()


def test_version_string_without_gpu():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    lib.al_version.restype = ctypes.c_char_p
    assert lib.al_version().decode().startswith("arclight_amd")


def test_struct_layouts_match_c(tmp_path):
    """Compiles a probe with the host C compiler that prints sizeof/offsetof
    of the public structs and compares with the ctypes mirrors."""
    src = tmp_path / "probe.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "arclight_fattn.h"\n'
        "int main(void) {\n"
        ' printf("%zu %zu %zu %zu\\n", sizeof(al_tensor), offsetof(al_tensor, ne), offsetof(al_tensor, nb),'
        " offsetof(al_tensor, data));\n"
        ' printf("%zu %zu %zu %zu %zu %zu %zu\\n", sizeof(al_fattn_args), offsetof(al_fattn_args, scale),'
        " offsetof(al_fattn_args, prec), offsetof(al_fattn_args, kv_len), offsetof(al_fattn_args, causal_pos0),"
        " offsetof(al_fattn_args, stream), offsetof(al_fattn_args, workspace_bytes));\n"
        " return 0; }\n")
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [list(map(int, line.split())) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                                     check=True).stdout.splitlines()]
    T, A = abi.AlTensor, abi.AlFattnArgs
    assert got[0] == [ctypes.sizeof(T), T.ne.offset, T.nb.offset, T.data.offset]
    assert got[1] == [ctypes.sizeof(A), A.scale.offset, A.prec.offset, A.kv_len.offset, A.causal_pos0.offset,
                      A.stream.offset, A.workspace_bytes.offset]


def test_attn_inputs_layout_matches_c(tmp_path):
    """al_attn_inputs_args (arclight_prologue.h) against its ctypes mirror,
    and al_fattn_args.dyn_len, the last field the graph-replay path adds."""
    src = tmp_path / "probe2.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "arclight_prologue.h"\n'
        "int main(void) {\n"
        ' printf("%zu %zu %zu %zu %zu\\n", sizeof(al_attn_inputs_args), offsetof(al_attn_inputs_args, v),'
        " offsetof(al_attn_inputs_args, v_cache), offsetof(al_attn_inputs_args, eps),"
        " offsetof(al_attn_inputs_args, rope));\n"
        ' printf("%zu %zu\\n", sizeof(al_fattn_args), offsetof(al_fattn_args, dyn_len));\n'
        " return 0; }\n")
    exe = tmp_path / "probe2"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [list(map(int, line.split())) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                                     check=True).stdout.splitlines()]
    I, A = abi.AlAttnInputsArgs, abi.AlFattnArgs
    assert got[0] == [ctypes.sizeof(I), I.v.offset, I.v_cache.offset, I.eps.offset, I.rope.offset]
    assert got[1] == [ctypes.sizeof(A), A.dyn_len.offset]


def test_attn_inputs_rejects_missing_operands_without_gpu():
    """Argument checks run before any device call: no arguments, and a Q
    tensor of the wrong type, come back as AL_ERR_INVALID / UNSUPPORTED."""
    from arclight_amd import _lib
    lib = _lib.load()
    assert lib.al_attn_inputs_f32(None, None) == abi.AL_ERR_INVALID
    a = abi.AlAttnInputsArgs()                     # every tensor empty
    assert lib.al_attn_inputs_f32(ctypes.byref(a), None) in (abi.AL_ERR_INVALID, abi.AL_ERR_UNSUPPORTED)
