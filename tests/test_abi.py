"""The C-ABI library: loads, exports every declared symbol, struct layout agrees (no GPU calls)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from tree_attention import _native

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tree_attn.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ta_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    names = declared_functions()
    assert set(names) == set(_native.EXPORTS)
    for name in names:
        assert hasattr(lib, name), name
    assert lib.ta_version().decode().startswith("tree_attn gfx950")
    assert b"16-byte" in lib.ta_error_string(1002)


def test_library_rejects_bad_arguments_without_gpu_work():
    lib = _native.load()
    # unsupported head dim / dtype / null pointers are refused before any launch
    assert lib.ta_merge(None, None, None, None, None, 1, 32, 96, 1, 0, None) == 1001
    assert lib.ta_merge(None, None, None, None, None, 1, 32, 128, 1, 7, None) == 1003
    assert lib.ta_segment(None, None, None, None, None, None, None, None, None, 1, 0, None, None,
                          1, 32, 8, 128, 16, 1, 0, None) == 1001
    assert lib.ta_segment(None, None, None, None, None, None, None, None, None, 1, 0, None, None,
                          1, 30, 8, 128, 16, 1, 0, None) == 1001
    assert lib.ta_attention_matrix(None, None, None, 1, None, None, None) == 1001
    # the timing hook takes both events or neither; NULL/NULL clears it
    assert lib.ta_time_next_launch(None, None) == 0
    assert lib.ta_time_next_launch(ctypes.c_void_p(16), None) == 1001


def test_plan_struct_layout_matches_header(tmp_path):
    fields = [f[0] for f in _native.TaPlan._fields_]
    src = tmp_path / "layout.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){",
             'printf("%zu\\n", sizeof(ta_plan));']
    lines += [f'printf("%zu\\n", offsetof(ta_plan, {f}));' for f in fields]
    lines.append("return 0;}")
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got[0] == ctypes.sizeof(_native.TaPlan)
    assert got[1:] == [getattr(_native.TaPlan, f).offset for f in fields]


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not found"):
        _native.load(tmp_path / "nope.so")


def test_xtail_record_layout_matches_header():
    """kernels.XTAIL_MAX and the record stride prepare writes equal TA_XTAIL_MAX / TA_XTAIL_STRIDE."""
    import re
    from pathlib import Path
    from tree_attention import kernels
    header = (Path(__file__).resolve().parents[1] / "include" / "tree_attn.h").read_text()
    assert int(re.search(r"#define TA_XTAIL_MAX (\d+)", header).group(1)) == kernels.XTAIL_MAX
    assert "#define TA_XTAIL_STRIDE (1 + 4 * TA_XTAIL_MAX)" in header
    assert kernels.XTAIL_FIELDS == 4


def test_python_constants_match_header():
    """Every constant _native mirrors equals its #define in include/tree_attn.h."""
    header = HEADER.read_text()

    def define(name):
        m = re.search(rf"#define {name} \(?(\d+)u?(?: << (\d+))?\)?", header)
        assert m, name
        return int(m.group(1)) << int(m.group(2) or 0)

    assert define("TA_NOALLOC_SCRATCH_BYTES") == _native.NOALLOC_SCRATCH_BYTES == 32 << 20
    assert define("TA_ERR_SCRATCH") == _native.TA_ERR_SCRATCH
    assert define("TA_ERR_ARG") == _native.TA_ERR_ARG
    for name in ("TA_BF16", "TA_FP16", "TA_SMALL", "TA_LARGE64", "TA_LARGE128", "TA_LARGE256", "TA_TAIL",
                 "TA_NKINDS"):
        assert define(name) == getattr(_native, name), name


def test_decode_append_rejects_host_slots_outside_the_pool():
    """Slots given as host data are range-checked before any launch (the eager
    index_copy_ of the reference adapter, qwen.py:89-90, raises for them too)."""
    import torch
    from tree_attention.kernels import decode_append
    nreq, hq, hk, d, tcap = 3, 8, 2, 32, 16
    q = torch.zeros(nreq, 1, hq, d, dtype=torch.bfloat16)
    k = torch.zeros(nreq, 1, hk, d, dtype=torch.bfloat16)
    v = torch.zeros(nreq, 1, hk, d, dtype=torch.bfloat16)
    cos = torch.ones(nreq, 1, d, dtype=torch.bfloat16)
    sin = torch.zeros(nreq, 1, d, dtype=torch.bfloat16)
    kp = torch.zeros(hk, d, tcap, dtype=torch.bfloat16)
    vp = torch.zeros(hk, tcap, d, dtype=torch.bfloat16)
    for bad in ([0, 5, tcap], [-1, 2, 3], torch.tensor([1, 2, tcap + 7])):
        with pytest.raises(ValueError, match="pool capacity"):
            decode_append(q, k, v, cos, sin, bad, kp, vp)
    with pytest.raises(ValueError, match="one pool position per request"):
        decode_append(q, k, v, cos, sin, [0, 1], kp, vp)
