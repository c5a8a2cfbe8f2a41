"""The C ABI library loads on a machine without a GPU, exports every entry point include/kda355.h declares, and
rejects invalid arguments with KDA355_EINVAL before touching the device."""
import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def _declared():
    text = (ROOT / "include" / "kda355.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(kda355_\w+)\s*\(", text, re.M)))


def test_header_lists_entry_points():
    names = _declared()
    assert "kda355_recurrent_launch" in names and "kda355_last_error" in names


def test_library_exports_every_declared_symbol():
    from kda355 import _lib
    L = _lib.lib()
    missing = [n for n in _declared() if not hasattr(L, n)]
    assert not missing, f"not exported: {missing}"
    assert L.kda355_version() >= 100


def test_invalid_arguments_rejected_without_gpu():
    from kda355 import _lib
    L = _lib.lib()
    a = _lib.KdaRecurrentArgs()
    a.B, a.S, a.H = 4, 1, 2                              # pointers left null
    assert L.kda355_recurrent_launch(ctypes.byref(a), None) == _lib.EINVAL
    assert b"null" in L.kda355_last_error()
    a.S = 0
    assert L.kda355_recurrent_launch(ctypes.byref(a), None) == _lib.EINVAL
    c = _lib.KdaSpecCommitArgs()
    c.B, c.S, c.H = 2, 2, 1
    assert L.kda355_spec_commit_launch(ctypes.byref(c), None) == _lib.EINVAL


def test_struct_layout_matches_header():
    """ctypes mirrors of the argument structs have the size the C compiler gives them."""
    import subprocess
    import tempfile
    from kda355 import _lib
    src = '#include "kda355.h"\n#include <stdio.h>\nint main(){printf("%zu %zu\\n", sizeof(KdaRecurrentArgs), ' \
          'sizeof(KdaSpecCommitArgs));return 0;}\n'
    with tempfile.TemporaryDirectory() as d:
        (Path(d) / "m.c").write_text(src)
        subprocess.run(["gcc", "-I", str(ROOT / "include"), str(Path(d) / "m.c"), "-o", str(Path(d) / "m")],
                       check=True)
        sizes = subprocess.run([str(Path(d) / "m")], capture_output=True, text=True, check=True).stdout.split()
    assert int(sizes[0]) == ctypes.sizeof(_lib.KdaRecurrentArgs)
    assert int(sizes[1]) == ctypes.sizeof(_lib.KdaSpecCommitArgs)
