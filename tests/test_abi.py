"""The boundary: the built library loads and exports exactly what
include/ditch_hip.h declares (no GPU needed, no compute calls)."""
import ctypes
import os

import pytest

import ditch_amd
from ditch_amd import abi


def test_header_declares_every_bound_prototype():
    declared = set(abi.header_symbols(ditch_amd.HEADER_PATH))
    assert declared == set(abi.PROTOTYPES), declared ^ set(abi.PROTOTYPES)


def test_library_exports_every_declared_symbol():
    if not os.path.exists(ditch_amd.LIB_PATH):
        pytest.fail("libditch_hip.so is not built (run python -m ditch_amd.build)")
    lib = ditch_amd.load_library()
    for name in abi.header_symbols(ditch_amd.HEADER_PATH):
        assert hasattr(lib, name), name


def test_struct_layouts_match_the_header():
    """Sizes of the ABI structs as compiled by the C compiler (gcc on the header)."""
    import subprocess
    import tempfile
    src = """
#include <stdio.h>
#include <stddef.h>
#include "ditch_hip.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\\n", sizeof(ditch_weight), sizeof(ditch_model_config), sizeof(ditch_row),
         offsetof(ditch_model_config, moe_layers), offsetof(ditch_weight, g_idx), sizeof(ditch_expert_cache_stats),
         sizeof(ditch_edit_options), offsetof(ditch_edit_options, seed), sizeof(ditch_model_path_stats),
         sizeof(ditch_residency_stats), sizeof(ditch_hot_expert), sizeof(ditch_edit_target),
         offsetof(ditch_edit_target, v), sizeof(ditch_sampler), offsetof(ditch_sampler, rng));
  return 0;
}
"""
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "t.c")
        open(c, "w").write(src)
        exe = os.path.join(d, "t")
        subprocess.run(["gcc", "-I", os.path.dirname(ditch_amd.HEADER_PATH), c, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()
    got = [int(v) for v in out]
    assert got == [ctypes.sizeof(abi.Weight), ctypes.sizeof(abi.ModelConfig), ctypes.sizeof(abi.Row),
                   abi.ModelConfig.moe_layers.offset, abi.Weight.g_idx.offset, ctypes.sizeof(abi.ExpertCacheStats),
                   ctypes.sizeof(abi.EditOptions), abi.EditOptions.seed.offset, ctypes.sizeof(abi.PathStats),
                   ctypes.sizeof(abi.ResidencyStats), ctypes.sizeof(abi.HotExpert), ctypes.sizeof(abi.EditTarget),
                   abi.EditTarget.v.offset, ctypes.sizeof(abi.Sampler), abi.Sampler.rng.offset]


def test_open_without_a_gpu_fails_cleanly():
    """No device: open returns NULL with a message; nothing aborts."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = ditch_amd.load_library()
    err = ctypes.create_string_buffer(256)
    assert not lib.ditch_hip_open(0, err, 256)
    assert err.value
    # every entry point is safe with a NULL context
    assert lib.ditch_hip_sync(None) == abi.INVALID_ARGUMENT
    assert lib.ditch_hip_matmulT(None, None, None, 0, None) == abi.INVALID_ARGUMENT
