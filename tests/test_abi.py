"""Host-side checks of the C ABI that need no GPU: the library loads, exports every entry point the header
declares, its struct layouts match the header as a C compiler sees it, and argument validation answers
with the documented statuses before any device work is enqueued."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from sharplight_amd import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sharplight_hip.h")


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"SLHIP_API\s+[\w\s\*]+?\b(slhip_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = native.lib()
    names = header_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert set(names) == set(native.SIGNATURES), set(names) ^ set(native.SIGNATURES)


def test_abi_version_matches_header():
    v = int(re.search(r"#define SLHIP_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert native.lib().slhip_abi_version() == v


def _c_layout():
    src = r"""
#include <stdio.h>
#include <stddef.h>
#include "sharplight_hip.h"
#define P(s, f) printf(#s "." #f " %zu\n", offsetof(s, f));
int main(void) {
  printf("slhip_device_props %zu\n", sizeof(slhip_device_props));
  printf("slhip_rope_tensor %zu\n", sizeof(slhip_rope_tensor));
  printf("slhip_rope_cfg %zu\n", sizeof(slhip_rope_cfg));
  printf("slhip_cache_rows %zu\n", sizeof(slhip_cache_rows));
  printf("slhip_norm_copies %zu\n", sizeof(slhip_norm_copies));
  P(slhip_norm_copies, y16_stride) P(slhip_norm_copies, yq) P(slhip_norm_copies, yq_stride)
  P(slhip_device_props, total_memory) P(slhip_device_props, l2_bytes) P(slhip_device_props, lds_bytes_per_block)
  P(slhip_rope_tensor, heads) P(slhip_rope_tensor, y_stride_h)
  P(slhip_rope_cfg, eps) P(slhip_rope_cfg, norm) P(slhip_rope_cfg, sections) P(slhip_rope_cfg, per_element)
  P(slhip_rope_tensor, rows)
  P(slhip_cache_rows, ctx) P(slhip_cache_rows, n_past) P(slhip_cache_rows, seq) P(slhip_cache_rows, slots)
  P(slhip_cache_rows, pages) P(slhip_cache_rows, page_slots) P(slhip_cache_rows, blocks_per_slot)
  P(slhip_cache_rows, block_size)
  return 0;
}
"""
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "l.c")
        exe = os.path.join(d, "l")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), c, "-o", exe],
                       check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    return dict(line.split() for line in out.strip().splitlines())


def test_struct_layouts_match_c():
    lay = {k: int(v) for k, v in _c_layout().items()}
    assert lay["slhip_device_props"] == ctypes.sizeof(native.DeviceProps)
    assert lay["slhip_rope_tensor"] == ctypes.sizeof(native.RopeTensor)
    assert lay["slhip_rope_cfg"] == ctypes.sizeof(native.RopeCfg)
    assert lay["slhip_device_props.total_memory"] == native.DeviceProps.total_memory.offset
    assert lay["slhip_device_props.l2_bytes"] == native.DeviceProps.l2_bytes.offset
    assert lay["slhip_device_props.lds_bytes_per_block"] == native.DeviceProps.lds_bytes_per_block.offset
    assert lay["slhip_rope_tensor.heads"] == native.RopeTensor.heads.offset
    assert lay["slhip_rope_tensor.y_stride_h"] == native.RopeTensor.y_stride_h.offset
    assert lay["slhip_rope_cfg.eps"] == native.RopeCfg.eps.offset
    assert lay["slhip_rope_cfg.norm"] == native.RopeCfg.norm.offset
    assert lay["slhip_rope_cfg.sections"] == native.RopeCfg.sections.offset
    assert lay["slhip_rope_cfg.per_element"] == native.RopeCfg.per_element.offset
    assert lay["slhip_cache_rows"] == ctypes.sizeof(native.CacheRows)
    assert lay["slhip_rope_tensor.rows"] == native.RopeTensor.rows.offset
    for f in ("ctx", "n_past", "seq", "slots", "pages", "page_slots", "blocks_per_slot", "block_size"):
        assert lay[f"slhip_cache_rows.{f}"] == getattr(native.CacheRows, f).offset, f
    assert lay["slhip_norm_copies"] == ctypes.sizeof(native.NormCopies)
    for f in ("y16_stride", "yq", "yq_stride"):
        assert lay[f"slhip_norm_copies.{f}"] == getattr(native.NormCopies, f).offset, f


# ---- argument validation (returns before touching the device) ------------------------------------------

FAKE = 0x1000  # never dereferenced: every call below fails validation first


def test_rownorm_validation():
    with pytest.raises(native.SlhipArgumentError, match="x and y"):
        native.rownorm("rms", "f32", "f32", None, None, 4, 8)
    with pytest.raises(native.SlhipArgumentError, match="bad kind"):
        native.rownorm(7, "f32", "f32", FAKE, FAKE, 4, 8)
    with pytest.raises(native.SlhipArgumentError, match="L2Norm"):
        native.rownorm("l2", "f32", "f32", FAKE, FAKE, 4, 8, w=FAKE)
    with pytest.raises(native.SlhipArgumentError, match="bias"):
        native.rownorm("rms", "f32", "f32", FAKE, FAKE, 4, 8, b=FAKE)
    with pytest.raises(native.SlhipArgumentError, match="stride"):
        native.rownorm("rms", "f32", "f32", FAKE, FAKE, 4, 8, x_stride=4)
    with pytest.raises(native.SlhipNotSupported):
        native.rownorm("rms", "f16", "f32", FAKE, FAKE, 4, 8)
    native.rownorm("rms", "f32", "f32", None, None, 0, 8)  # empty: nothing to do, no pointers needed


def test_rownorm_copies_validation():
    with pytest.raises(native.SlhipArgumentError, match="y or a copy"):
        native.call("slhip_rownorm_copies", 0, 0, 0, FAKE, None, None, None, None, None, 4, 128, 128, 128, 128, 128,
                    1e-6, None, None)
    with pytest.raises(native.SlhipArgumentError, match="multiple of 128"):
        native.rownorm("rms", "f32", "f32", FAKE, None, 4, 96, yq=FAKE)
    with pytest.raises(native.SlhipArgumentError, match=r"D \+ D/32 = 264"):
        native.rownorm("rms", "bf16", "bf16", FAKE, None, 4, 256, yq=FAKE, yq_stride=260)
    with pytest.raises(native.SlhipArgumentError, match="4-byte aligned"):
        native.rownorm("rms", "bf16", "bf16", FAKE, None, 4, 256, yq=FAKE + 2)
    with pytest.raises(native.SlhipArgumentError, match="stride"):
        native.rownorm("rms", "f32", "f32", FAKE, None, 4, 128, y16=FAKE, y16_stride=64)


def test_gated_validation():
    with pytest.raises(native.SlhipArgumentError):
        native.gated_act("silu", "bf16", "bf16", None, FAKE, FAKE, 2, 8)
    with pytest.raises(native.SlhipArgumentError, match="bad activation"):
        native.gated_act(9, "bf16", "bf16", FAKE, FAKE, FAKE, 2, 8)
    with pytest.raises(native.SlhipArgumentError, match="stride"):
        native.gated_act("silu", "bf16", "bf16", FAKE, FAKE, FAKE, 2, 8, gate_stride=4)
    native.gated_act("silu", "bf16", "bf16", None, None, None, 0, 8)


def test_rope_validation():
    t = [dict(x=FAKE, y=FAKE, heads=2)]
    with pytest.raises(native.SlhipArgumentError, match="dims"):
        native.rope("f32", "f32", t, FAKE, 4, 16, dims=18)
    with pytest.raises(native.SlhipArgumentError, match="dims"):
        native.rope("f32", "f32", t, FAKE, 4, 16, dims=7)
    with pytest.raises(native.SlhipArgumentError, match="positions"):
        native.rope("f32", "f32", t, None, 4, 16)
    with pytest.raises(native.SlhipArgumentError, match="between 1 and 4"):
        native.rope("f32", "f32", t * 5, FAKE, 4, 16)
    with pytest.raises(native.SlhipArgumentError, match="norm weight"):
        native.rope("f32", "f32", [dict(x=FAKE, y=FAKE, heads=2, norm_w=FAKE)], FAKE, 4, 16)
    with pytest.raises(native.SlhipNotSupported):
        native.rope("f16", "f32", t, FAKE, 4, 16)


def test_gather_validation():
    with pytest.raises(native.SlhipNotSupported, match="format"):
        native.gather(99, FAKE, 10, 32, FAKE, 4, "bf16", FAKE)
    with pytest.raises(native.SlhipArgumentError, match="block size"):
        native.gather("q8_0", FAKE, 10, 40, FAKE, 4, "bf16", FAKE)
    with pytest.raises(native.SlhipArgumentError, match="null"):
        native.gather("q4_0", None, 10, 64, FAKE, 4, "bf16", FAKE)
    with pytest.raises(native.SlhipNotSupported, match="output dtype"):
        native.gather("q4_0", FAKE, 10, 64, FAKE, 4, "f16", FAKE)
    native.gather("q8_0", None, 10, 32, None, 0, "bf16", None)


def test_last_error_is_thread_local_and_never_null():
    import threading
    with pytest.raises(native.SlhipArgumentError):
        native.rownorm("rms", "f32", "f32", None, None, 4, 8)
    seen = []
    th = threading.Thread(target=lambda: seen.append(native.last_error()))
    th.start()
    th.join()
    assert seen == [""]
    assert "x and y" in native.last_error()


def test_matvec_validation():
    with pytest.raises(native.SlhipArgumentError, match="null"):
        native.matvec("bf16", "f32", "f32", None, 1, 64, FAKE, 4, FAKE)
    with pytest.raises(native.SlhipArgumentError, match="bad activation"):
        native.dual_matvec(7, "bf16", "f32", "f32", FAKE, 1, 64, FAKE, FAKE, 4, FAKE)
    with pytest.raises(native.SlhipNotSupported, match="weight format"):
        native.matvec(42, "f32", "f32", FAKE, 1, 64, FAKE, 4, FAKE)
    with pytest.raises(native.SlhipNotSupported, match="multiple of 256"):
        native.matvec("q4_1", "f32", "f32", FAKE, 1, 128, FAKE, 4, FAKE)
    with pytest.raises(native.SlhipNotSupported, match="multiple of 8"):
        native.matvec("bf16", "f32", "f32", FAKE, 1, 60, FAKE, 4, FAKE)
    with pytest.raises(native.SlhipNotSupported, match="16384"):
        native.matvec("bf16", "f32", "f32", FAKE, 1, 16392, FAKE, 4, FAKE)
    with pytest.raises(native.SlhipArgumentError, match="stride"):
        native.matvec("bf16", "f32", "f32", FAKE, 1, 64, FAKE, 4, FAKE, x_stride=32)
    with pytest.raises(native.SlhipNotSupported, match="f32 or bf16"):
        native.matvec("bf16", "f16", "f32", FAKE, 1, 64, FAKE, 4, FAKE)
