"""The C-ABI library (CPU only): it loads, exports every function the public
header declares, the Python binding describes each of them, and argument
validation fails cleanly without touching a GPU."""

import ctypes
import re
from pathlib import Path

import pytest

from mirai_amd import _native as nat

HEADER = Path(__file__).resolve().parents[1] / "include" / "mirai_moe.h"


def _declared() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mx_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not nat.LIB_PATH.exists():
        pytest.fail(f"{nat.LIB_PATH} is not built; run __graft_entry__.build()")
    return nat.load_library()


def test_header_declares_the_entry_points():
    names = _declared()
    for required in ("mx_route_topk", "mx_build_plan", "mx_moe_forward", "mx_moe_backward",
                     "mx_combine", "mx_nf4_quantize", "mx_int8_dequantize", "mx_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, f"declared in mirai_moe.h but not exported: {missing}"


def test_binding_covers_every_declared_symbol():
    assert sorted(nat.SIGNATURES) == _declared()


def test_abi_version_and_error_text(lib):
    assert lib.mx_abi_version() == 9
    assert isinstance(nat.last_error(), str)


def test_workspace_sizes(lib):
    assert lib.mx_moe_workspace_size(4096, 4, 64, 2048, 1408, 32) > 0
    assert lib.mx_moe_backward_workspace_size(8192, 4, 64, 2048, 1408, 32) > 0
    assert lib.mx_plan_workspace_size(1000, 4, 64) > 0
    assert lib.mx_moe_workspace_size(-1, 4, 64, 2048, 1408, 32) == 0
    assert lib.mx_moe_backward_workspace_size(16, 0, 64, 2048, 1408, 32) == 0
    # Grows with the problem.
    assert lib.mx_moe_workspace_size(8192, 4, 64, 2048, 1408, 32) > lib.mx_moe_workspace_size(
        4096, 4, 64, 2048, 1408, 32)
    # The low-rank rows: 3 planes of max(32, rank rounded up to 32) bf16 columns.
    R = 4096 * 4
    base = lib.mx_moe_workspace_size(4096, 4, 64, 2048, 1408, 0)
    assert lib.mx_moe_workspace_size(4096, 4, 64, 2048, 1408, 32) == base
    assert lib.mx_moe_workspace_size(4096, 4, 64, 2048, 1408, 48) == base + R * 3 * 32 * 2
    assert lib.mx_moe_workspace_size(4096, 4, 64, 2048, 1408, 256) == base + R * 3 * 224 * 2
    assert lib.mx_moe_workspace_size(4096, 4, 64, 2048, 1408, 264) == 0
    assert lib.mx_moe_backward_workspace_size(4096, 4, 64, 2048, 1408, -8) == 0
    assert (lib.mx_moe_backward_workspace_size(4096, 4, 64, 2048, 1408, 64)
            > lib.mx_moe_backward_workspace_size(4096, 4, 64, 2048, 1408, 32))
    assert (lib.mx_moe_expert_choice_workspace_size(2, 8, 16, 64, 8, 256, 192, 128)
            > lib.mx_moe_expert_choice_workspace_size(2, 8, 16, 64, 8, 256, 192, 0) > 0)
    assert (lib.mx_moe_backward_expert_choice_workspace_size(2, 8, 16, 64, 8, 256, 192, 128)
            > lib.mx_moe_backward_expert_choice_workspace_size(2, 8, 16, 64, 8, 256, 192, 8) > 0)


def _rc(name, *args):
    return getattr(nat.load_library(), name)(*args)


def test_validation_errors_return_invalid_without_a_gpu():
    null = None
    assert _rc("mx_route_topk", null, 8, 4, 9, 1, 1.0, null, null, 0, null) == 1  # k > E
    assert "mx_route_topk" in nat.last_error()
    assert _rc("mx_nf4_quantize", null, 1, 4, 96, null, null, null) == 1  # cols % 64
    assert _rc("mx_build_plan", null, null, 0, 8, 0, 4, *([null] * 9)) == 1  # k = 0
    w = nat.MxWeight(2, None, None, 1408, 2048)
    lora = nat.MxLora(None, None, 0, 0.0)
    rc = _rc("mx_moe_forward", null, null, null, 0, 16, 4, 8, 100, 1408, ctypes.byref(w),
             ctypes.byref(w), ctypes.byref(w), ctypes.byref(lora), ctypes.byref(lora),
             ctypes.byref(lora), null, 1, null, null, null, null, null, null, null)
    assert rc == 1 and "multiples of 64" in nat.last_error()
    bad_rank = nat.MxLora(1, 1, 12, 1.0)
    w1 = nat.MxWeight(2, 1, 1, 128, 64)
    w2 = nat.MxWeight(2, 1, 1, 64, 128)
    rc = _rc("mx_moe_backward", null, 1, null, null, null, 0, 16, 4, 8, 64, 128,
             ctypes.byref(w1), ctypes.byref(w1), ctypes.byref(w2), ctypes.byref(bad_rank),
             ctypes.byref(lora), ctypes.byref(lora), *([null] * 5), null, 1, null,
             *([null] * 6), null, null)
    assert rc == 1 and "rank" in nat.last_error()


def test_call_maps_codes_to_python_exceptions():
    with pytest.raises(ValueError, match="mx_route_topk"):
        nat.call("mx_route_topk", None, 8, 4, 9, 1, 1.0, None, None, 0, None)


def test_struct_layouts_match_the_header(tmp_path):
    # The ctypes mirrors of the header's structs: sizes and field offsets as a C
    # compiler lays them out (gcc on the header itself, no GPU involved).
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    structs = {"mx_weight": nat.MxWeight, "mx_lora": nat.MxLora, "mx_nf4_dq": nat.MxNf4Dq}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"',
             "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'  printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    # The header declares hipStream_t-free C; it only needs stdint / stddef.
    subprocess.run([cc, "-std=c11", "-o", str(exe), str(src)], check=True, capture_output=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    got = {}
    for line in out.splitlines():
        name, key, val = line.split()
        got[(name, key)] = int(val)
    for cname, py in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for field, _ in py._fields_:
            assert got[(cname, field)] == getattr(py, field).offset, (cname, field)
