# SPDX-License-Identifier: Apache-2.0
"""dsv4_hip_load_experts rejects a bad checkpoint before it touches the
device: these run on the CPU (no GPU call is reached)."""
import os
import struct

import pytest

from ckpt_writer import write_checkpoint


@pytest.fixture
def lib(pkg):
    return pkg.load()


def test_bad_magic(lib, tmp_path):
    (tmp_path / "model").mkdir()
    (tmp_path / "model" / "a.safetensors").write_bytes(b"\0" * 64)
    (tmp_path / "experts.idx").write_bytes(b"DSV4XXXX" + struct.pack("<ii", 1, 1))
    with pytest.raises(Exception, match="DSV4EXP1"):
        lib.load_experts(str(tmp_path / "model"), str(tmp_path), 0, 512, 256)


def test_layer_out_of_range_and_short_index(lib, tmp_path):
    (tmp_path / "model").mkdir()
    (tmp_path / "model" / "a.safetensors").write_bytes(b"\0" * 64)
    (tmp_path / "experts.idx").write_bytes(b"DSV4EXP1" + struct.pack("<ii", 2, 4) + b"\0" * 24)
    with pytest.raises(Exception, match="layer 2 outside"):
        lib.load_experts(str(tmp_path / "model"), str(tmp_path), 2, 512, 256)
    with pytest.raises(Exception, match="short for layer 1"):
        lib.load_experts(str(tmp_path / "model"), str(tmp_path), 1, 512, 256)


def test_wrong_tensor_size_and_no_shards(lib, oracle, tmp_path):
    model_dir, index_dir, _ = write_checkpoint(oracle, str(tmp_path), 1, 2, 256, 128, seed=3)
    # the index was written for hidden 256 / inter 128: other geometries are rejected
    with pytest.raises(Exception, match="want"):
        lib.load_experts(model_dir, index_dir, 0, 512, 128)
    empty = tmp_path / "empty"
    empty.mkdir()
    with pytest.raises(Exception, match="no .safetensors"):
        lib.load_experts(str(empty), index_dir, 0, 256, 128)


def test_table_too_small(lib, oracle, tmp_path):
    model_dir, index_dir, _ = write_checkpoint(oracle, str(tmp_path), 1, 3, 256, 128, seed=4)
    with pytest.raises(Exception, match="table holds 2"):
        lib.load_experts(model_dir, index_dir, 0, 256, 128, max_experts=2)
