"""CPU-side checks of the product library and host logic (no GPU calls)."""
import ctypes
import os

import numpy as np
import pytest

import qtts
from qtts import hostdesc, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(qtts.LIB_PATH)
    declared = qtts.header_symbols()
    assert len(declared) >= 30
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, f"declared in include/qtts.h but not exported: {missing}"
    assert set(qtts.SIGNATURES) == set(declared), "binding signatures out of step with the header"


def test_binding_loads_and_types():
    lib = qtts.load_library()
    assert lib.qtts_ctx_create.restype is ctypes.c_int


def test_struct_layouts_match_header():
    # offsets of the C structs as laid out by the C compiler (x86-64 SysV)
    assert ctypes.sizeof(hostdesc.Q4Host) == 32
    assert ctypes.sizeof(hostdesc.LayerHost) == 7 * 32 + 4 * 8
    assert hostdesc.TalkerHost.layers.offset == 32
    assert ctypes.sizeof(hostdesc.SampleParams) == 32


def test_synth_shapes_and_determinism():
    t1 = synth.make_talker(seed=3, n_layers=1, text_vocab=16, rope_max_pos=8)
    t2 = synth.make_talker(seed=3, n_layers=1, text_vocab=16, rope_max_pos=8)
    L = t1.layers[0]
    assert L.q_proj.packed.shape == (2048, 1024) and L.q_proj.scales.shape == (2048, 64)
    assert L.gate_proj.k == 2048 and L.gate_proj.n == 6144 and L.down_proj.k == 6144
    assert np.array_equal(L.up_proj.packed, t2.layers[0].up_proj.packed)
    s = L.q_proj.scales.view(np.float16).astype(np.float32)
    assert s.min() >= 0 and 0.01 < s.mean() < 0.02      # |N(0, 0.02)|: mean 0.016
    nib = np.concatenate([(L.q_proj.packed & 15).ravel(), (L.q_proj.packed >> 4).ravel()])
    assert nib.min() == 0 and nib.max() == 15


def test_missing_library_raises(tmp_path):
    with pytest.raises(qtts.QttsError):
        qtts.load_library(str(tmp_path / "nope.so"))


def test_tile_shapes_match_device_table():
    """qtts.TILE_SHAPES mirrors tile_shape() in csrc/qtts_device.h."""
    import re
    src = open(os.path.join(ROOT, "qora-tts-12hz-1.7b_amd", "csrc", "qtts_device.h")).read()
    body = src[src.index("constexpr TileShape tab[TILE_COUNT]"):]
    body = body[body.index("{") + 1: body.index("};")]
    tab = [tuple(int(v) for v in m) for m in re.findall(r"\{(\d+),\s*(\d+),\s*(\d+)\}", body)]
    assert tab == qtts.TILE_SHAPES
    n_enum = len(re.findall(r"^\s*TILE_G\d+_T\d+(?:_R\d)?\s*=\s*\d+", src, re.M))
    assert n_enum == len(tab)


def test_icl_layout_known_answers():
    """icl_block_layout's own tests (generate_new.rs:869-900) through the
    host-only export."""
    assert qtts.icl_layout(8, 8, 23) == (24, 0)      # text shorter: pad branch
    assert qtts.icl_layout(30, 30, 23) == (24, 37)   # text longer: remainder
    assert qtts.icl_layout(11, 11, 22) == (23, 0)    # equal lengths
    assert qtts.icl_layout(1, 1, 23) == (24, 0)      # short reference
    with pytest.raises(qtts.QttsError):
        qtts.icl_layout(1, 1, 0)


def test_prefix_suffix_split_known_answers():
    """prefix_suffix_split's own tests (generate_new.rs:986-1001)."""
    assert qtts.prefix_suffix_split(162, 35, 44) == 127
    assert qtts.prefix_suffix_split(162, 35, 43) is None   # prefix length mismatch
    assert qtts.prefix_suffix_split(35, 35, 44) is None    # empty suffix
    assert qtts.prefix_suffix_split(30, 35, 44) is None    # block shorter than the reference
    assert qtts.prefix_suffix_split(162, 0, 9) == 162
