"""The C-ABI without a GPU: libtdgs.so loads, exports every function include/tdgs.h
declares, its argument validation reports errors through the status code and
tdgs_last_error(), and the ctypes struct mirrors match the C layouts (sizes and offsets as
compiled by gcc from the header)."""
import ctypes as C
import os
import re
import subprocess

import pytest

from conftest import ROOT
from tdgs_amd import abi

HEADER = os.path.join(ROOT, "include", "tdgs.h")
LIB = os.path.join(ROOT, "threedgaussiansplatting.jl_amd", "libtdgs.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tdgs_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        import __graft_entry__
        __graft_entry__.build()
    L = C.CDLL(LIB)
    L.tdgs_last_error.restype = C.c_char_p
    return L


def test_every_declared_function_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\sT\s(tdgs_[a-z0-9_]+)", out))
    assert exported == set(names), (exported ^ set(names))


def test_abi_version(lib):
    assert lib.tdgs_abi_version() == 2


def test_argument_validation_without_gpu(lib):
    rc = lib.tdgs_sort_pairs(None, C.c_size_t(0), None, None, None, None, C.c_int32(10), C.c_int32(65), None)
    assert rc == abi.TDGS_ERR_INVALID
    assert b"end_bit" in lib.tdgs_last_error()
    rc = lib.tdgs_sh_resize(None, None, C.c_int32(4), None, C.c_int32(17), C.c_int64(1), C.c_int32(1))
    assert rc == abi.TDGS_ERR_INVALID
    lib.tdgs_scan_temp_bytes.restype = C.c_size_t
    lib.tdgs_scan_temp_bytes.argtypes = [C.c_int64]
    assert lib.tdgs_scan_temp_bytes(2048 * 3 + 1) >= 4 * 8
    rc = lib.tdgs_render(None, None, None, None, None, None, None, None, None, None)
    assert rc == abi.TDGS_ERR_INVALID


STRUCTS = {
    "tdgs_camera": abi.Camera, "tdgs_render_options": abi.RenderOptionsC, "tdgs_tiling": abi.TilingC,
    "tdgs_gaussians": abi.Gaussians, "tdgs_render_buffers": abi.RenderBuffersC,
    "tdgs_render_outputs": abi.RenderOutputsC, "tdgs_gradients": abi.GradientsC,
    "tdgs_adam_state": abi.AdamStateC, "tdgs_adc_buffers": abi.AdcBuffersC,
}


def test_ctypes_mirrors_match_header_layout(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, py in STRUCTS.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", str(src), "-o", str(exe)], check=True)
    got = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                                 check=True).stdout.splitlines())
    for cname, py in STRUCTS.items():
        assert int(got[cname]) == C.sizeof(py), cname
        for fname, _ in py._fields_:
            assert int(got[f"{cname}.{fname}"]) == getattr(py, fname).offset, (cname, fname)


def test_new_entry_points_validate_without_gpu(lib):
    """Argument checks of tdgs_project, the stream/event plumbing, tdgs_ctx_check and the 2D
    gradient layouts run before any HIP call."""
    assert lib.tdgs_project(None, None, None, None, None, None, None, None) == abi.TDGS_ERR_INVALID
    assert lib.tdgs_stream_create(None) == abi.TDGS_ERR_INVALID
    assert lib.tdgs_stream_destroy(None) == abi.TDGS_ERR_INVALID
    assert lib.tdgs_event_create(None) == abi.TDGS_ERR_INVALID
    assert lib.tdgs_event_record(None, None) == abi.TDGS_ERR_INVALID
    assert lib.tdgs_stream_wait_event(None, None) == abi.TDGS_ERR_INVALID
    assert lib.tdgs_event_synchronize(None) == abi.TDGS_ERR_INVALID
    assert lib.tdgs_event_elapsed_ms(None, None, None) == abi.TDGS_ERR_INVALID
    assert lib.tdgs_host_malloc(None, C.c_size_t(16)) == abi.TDGS_ERR_INVALID
    assert lib.tdgs_ctx_check(None, None) == abi.TDGS_ERR_INVALID
    # backward blending with neither 2D gradient layout
    cam = abi.Camera(width=32, height=32)
    tiling = abi.TilingC(16, 16, 2, 2)
    opts = abi.RenderOptionsC(min_alpha=1 / 255, max_alpha=0.99, min_transmittance=1e-4)
    gr = abi.GradientsC(capacity=4, sh_degree=0)
    gr.mean2d_grads = 0x1000   # three of the four reference arrays only
    gr.opacity_grads = 0x1000
    gr.licov2d_grads = 0x1000
    dummy = C.c_void_p(0x1000)
    out = abi.RenderOutputsC(None, 0x1000, None, 0x1000)
    buf = abi.RenderBuffersC()
    rc = lib.tdgs_backward_render_tiles(None, C.byref(gr), dummy, C.byref(out), C.byref(cam), C.byref(tiling),
                                        C.byref(opts), C.byref(buf))
    assert rc == abi.TDGS_ERR_INVALID and b"color_grads" in lib.tdgs_last_error()
    # tiles of more than 1024 pixels
    big = abi.TilingC(40, 40, 1, 1)
    cam40 = abi.Camera(width=40, height=40)
    rc = lib.tdgs_render_tiles(None, C.byref(cam40), C.byref(big), C.byref(opts), C.byref(buf), C.byref(out))
    assert rc == abi.TDGS_ERR_INVALID and b"1024" in lib.tdgs_last_error()
