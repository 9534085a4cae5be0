"""The weight-file reader (prichs_checkpoint_*) against the reference's file
layout (crates/prichs-model/src/model.rs:1648-1736) and parameter order
(model.rs:312-338, 557-562, 1083-1087).  Host only: no GPU is needed.

Pins: a golden byte string typed from the format (header fields and one
tensor), bit-exact round trips including NaN payloads, signed zeros,
infinities and subnormals, and the block index map checked against an
enumeration of the reference's parameter list (not against its closed form).
"""
import struct

import numpy as np
import pytest

from prichs_amd import _lib as L
from prichs_amd import checkpoint as ck


def test_writer_and_reader_match_golden_bytes(tmp_path):
    # "PRICHS02", step 3 (u64), loss 1.0 (f32), 2 tensors: [2.0] and [].
    golden = bytes.fromhex("5052494348533032" "0300000000000000" "0000803f"
                           "0200000000000000" "0100000000000000" "00000040"
                           "0000000000000000")
    p = tmp_path / "golden.prichs"
    ck.write_prichs02(p, 3, 1.0, [np.array([2.0], np.float32), np.zeros(0, np.float32)])
    assert p.read_bytes() == golden
    with ck.Checkpoint(p) as c:
        assert (c.step, c.loss, c.n_params, c.format) == (3, 1.0, 2, 2)
        assert c.read(0).tolist() == [2.0]
        assert c.param_len(1) == 0 and c.read(1).size == 0


def test_reader_is_bit_exact(tmp_path):
    special = np.array([0x7FC00001, 0xFFC12345, 0x80000000, 0x00000000, 0x7F800000, 0xFF800000,
                        0x00000001, 0x007FFFFF, 0x7F7FFFFF], dtype=np.uint32).view(np.float32)
    rng = np.random.default_rng(7)
    tensors = [special, rng.standard_normal((33, 17)).astype(np.float32),
               rng.standard_normal(1).astype(np.float32)]
    p = tmp_path / "bits.prichs"
    ck.write_prichs02(p, 2**40 + 5, -0.5, tensors)
    with ck.Checkpoint(p) as c:
        assert c.step == 2**40 + 5 and c.loss == -0.5 and c.n_params == 3
        for i, t in enumerate(tensors):
            got = c.read(i)
            assert got.size == t.size
            np.testing.assert_array_equal(got.view(np.uint32), t.reshape(-1).view(np.uint32))


def _reference_parameter_names(n_blocks, E):
    # The push order of Model::get_parameter_tensors (model.rs:312-338).
    names = ["wte", "final_norm"]
    for l in range(n_blocks):
        names += [f"{l}.input_norm", f"{l}.q_proj", f"{l}.k_proj", f"{l}.v_proj",
                  f"{l}.out_proj", f"{l}.post_attn_norm", f"{l}.router",
                  f"{l}.shared.gate", f"{l}.shared.up", f"{l}.shared.down"]
        for e in range(E):
            names += [f"{l}.e{e}.gate", f"{l}.e{e}.up", f"{l}.e{e}.down"]
    return names


@pytest.mark.parametrize("E", [8, 3, 1])
def test_block_index_map_follows_parameter_order(E):
    names = _reference_parameter_names(3, E)
    slot_names = ["input_norm", "q_proj", "k_proj", "v_proj", "out_proj", "post_attn_norm",
                  "router", "shared.gate", "shared.up", "shared.down"]
    for e in range(E):
        slot_names += [f"e{e}.gate", f"e{e}.up", f"e{e}.down"]
    for l in range(3):
        for slot, nm in enumerate(slot_names):
            assert ck.block_param(l, E, slot) == names.index(f"{l}.{nm}")
    with pytest.raises(IndexError):
        ck.block_param(0, E, 10 + 3 * E)
    assert (ck.block_param(0, E, ck.EXPERT0 + 3 * (E - 1) + 2) ==
            names.index(f"0.e{E - 1}.down"))


def _expect_invalid(path):
    with pytest.raises(L.PrichsError) as e:
        ck.Checkpoint(path)
    assert e.value.status == L.PRICHS_ERR_INVALID_ARGUMENT
    return e.value.message


def test_malformed_files_fail_at_open(tmp_path):
    good = tmp_path / "good.prichs"
    ck.write_prichs02(good, 1, 0.0, [np.ones(8, np.float32), np.ones(4, np.float32)])
    raw = good.read_bytes()
    cases = {
        "magic": b"PRICHS03" + raw[8:],
        "short_header": raw[:10],
        "no_count": raw[:24],
        "count_too_large": raw[:20] + struct.pack("<Q", 10**6) + raw[28:],
        "payload_cut": raw[:-3],
        "length_cut": raw[:28 + 8 + 32 + 4],
    }
    for name, data in cases.items():
        p = tmp_path / f"{name}.prichs"
        p.write_bytes(data)
        msg = _expect_invalid(p)
        assert msg, name
    assert "cannot open" in _expect_invalid(tmp_path / "missing.prichs")
    # Trailing bytes after the last tensor are ignored, as the reference's
    # reader ignores them (it reads exactly what the header announces).
    p = tmp_path / "trailing.prichs"
    p.write_bytes(raw + b"\x00" * 5)
    with ck.Checkpoint(p) as c:
        assert c.n_params == 2 and c.read(1).tolist() == [1.0] * 4


def test_legacy_file_has_no_block_parameters(tmp_path):
    # PRICHS_W (model.rs:1707-1729): step, loss, total floats, wte, final_norm.
    p = tmp_path / "legacy.prichs"
    p.write_bytes(b"PRICHS_W" + struct.pack("<QfQ", 9, 2.5, 6) + np.arange(6, dtype="<f4").tobytes())
    with ck.Checkpoint(p) as c:
        assert (c.step, c.loss, c.n_params, c.format) == (9, 2.5, 0, 1)


def test_read_and_upload_argument_errors(tmp_path):
    p = tmp_path / "a.prichs"
    ck.write_prichs02(p, 0, 0.0, [np.ones(3, np.float32)])
    lib = L.load()
    with ck.Checkpoint(p) as c:
        with pytest.raises(L.PrichsError):
            L.check(lib.prichs_checkpoint_read(c.handle, 0, np.empty(4, np.float32).ctypes.data, 4))
        with pytest.raises(L.PrichsError):
            c.param_len(1)
        # Null engines are rejected before any HIP call (no GPU needed).
        assert lib.prichs_moe_engine_upload_checkpoint(None, c.handle, 0, None) == \
            L.PRICHS_ERR_INVALID_ARGUMENT
        assert lib.prichs_block_engine_upload_checkpoint(None, c.handle, 0, None) == \
            L.PRICHS_ERR_INVALID_ARGUMENT
    assert lib.prichs_checkpoint_close(None) == L.PRICHS_OK
