"""Weight files: momijo's checkpoint format (learn/utils/checkpoint.mojo:19-140,
learn/utils/tensor_bytes.mojo:40-85) and the MJW8 int8 file."""
import json
import struct

import numpy as np
import pytest

from momijo_amd import weights as wf


def test_make_checkpoint_header_and_order():
    W1 = np.arange(6, dtype=np.float32).reshape(2, 3)
    b1 = np.array([10, 11], np.float32)
    W2 = np.array([[20, 21]], np.float32)
    header, blob = wf.make_checkpoint([(W1, b1), (W2, None)])
    # the header string make_checkpoint builds (checkpoint.mojo:38-99)
    assert header == ('{"params":[{"type":"Linear","w":6,"b":2},'
                      '{"type":"Linear","w":2,"b":0}]}')
    np.testing.assert_array_equal(blob, [0, 1, 2, 3, 4, 5, 10, 11, 20, 21])
    back = wf.apply_checkpoint([((2, 3), True), ((1, 2), False)], header, blob)
    np.testing.assert_array_equal(back[0][0], W1)
    np.testing.assert_array_equal(back[0][1], b1)
    np.testing.assert_array_equal(back[1][0], W2)
    assert back[1][1].size == 0
    assert wf.apply_checkpoint([((4, 4), True)], header, blob) is None


def test_csv_round_trip_exact():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(500).astype(np.float32),
                        np.array([0.0, -0.0, 1e-45, 3.4028235e38, -1.17549435e-38,
                                  0.1, 1 / 3], np.float32)])
    y = wf.unpack_csv(wf.pack_csv(x))
    np.testing.assert_array_equal(y.view(np.uint32), x.view(np.uint32))


def test_csv_reader_rules():
    """Empty fields are skipped and unparsable ones read as 0.0
    (tensor_bytes.mojo:60-79)."""
    np.testing.assert_array_equal(wf.unpack_csv(b"1.5,,2,abc,3,"), [1.5, 2.0, 0.0, 3.0])
    assert wf.unpack_csv(b"").size == 0


def _entries(rng):
    out = []
    for i, (n, k, bias) in enumerate([(5, 40, True), (3, 7, False), (16, 256, True)]):
        q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
        s = rng.random(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32) if bias else None
        out.append(wf.W8Entry(f"l{i}", q, s, b, "rhe" if i % 2 == 0 else "legacy"))
    return out


def test_w8_round_trip(tmp_path):
    rng = np.random.default_rng(1)
    ents = _entries(rng)
    p = str(tmp_path / "m.mjw8")
    wf.save_w8(p, ents)
    back = wf.load_w8(p)
    assert [e.name for e in back] == [e.name for e in ents]
    for a, b in zip(ents, back):
        np.testing.assert_array_equal(a.q, b.q)
        np.testing.assert_array_equal(a.scales, b.scales)
        assert (a.bias is None) == (b.bias is None)
        if a.bias is not None:
            np.testing.assert_array_equal(a.bias, b.bias)
        assert a.rounding == b.rounding


def test_w8_sections_aligned(tmp_path):
    p = str(tmp_path / "m.mjw8")
    wf.save_w8(p, _entries(np.random.default_rng(2)))
    raw = open(p, "rb").read()
    assert raw[:4] == b"MJW8"
    ver, hlen, _ = struct.unpack("<III", raw[4:16])
    meta = json.loads(raw[16:16 + hlen])
    for L in meta["layers"]:
        for key in ("q", "scales", "bias"):
            if L[key] is not None:
                assert L[key][0] % 256 == 0 and L[key][0] >= 16 + hlen


def test_w8_rejects_corruption(tmp_path):
    p = str(tmp_path / "m.mjw8")
    wf.save_w8(p, _entries(np.random.default_rng(3)))
    raw = bytearray(open(p, "rb").read())
    hlen = struct.unpack("<III", bytes(raw[4:16]))[1]
    q0 = json.loads(bytes(raw[16:16 + hlen]))["layers"][0]["q"][0]
    bad = bytearray(raw)
    bad[q0 + 3] ^= 0xFF  # a byte of the first layer's int8 weights
    open(p, "wb").write(bytes(bad))
    with pytest.raises(ValueError, match="CRC"):
        wf.load_w8(p)
    bad = bytearray(raw)
    bad[0:4] = b"XXXX"
    open(p, "wb").write(bytes(bad))
    with pytest.raises(ValueError, match="not an MJW8"):
        wf.load_w8(p)
    open(p, "wb").write(bytes(raw[: len(raw) // 2]))
    with pytest.raises(ValueError):
        wf.load_w8(p)


@pytest.mark.gpu
def test_quantized_checkpoint_to_device(oracle, dev, tmp_path):
    """momijo fp32 checkpoint (CSV blob) -> per-channel int8 on the device ->
    MJW8 file -> W8Linear in HBM: q and scales bit-exact with the oracle's
    packing, and the layer computes what a layer quantized in memory does."""
    import torch
    import momijo_amd as mj
    W1 = oracle.randn_f32((96, 64), std=0.02, seed=5)
    b1 = oracle.randn_f32((96,), seed=6)
    W2 = oracle.randn_f32((32, 96), std=0.02, seed=7)
    header, blob = wf.make_checkpoint([(W1, b1), (W2, None)])
    blob2 = wf.unpack_csv(wf.pack_csv(blob))
    p = str(tmp_path / "q.mjw8")
    wf.quantize_checkpoint(header, blob2, [((96, 64), True), ((32, 96), False)], p, dev)
    layers = wf.load_w8(p, device=dev)
    for lin, W in zip(layers, (W1, W2)):
        q_ref, s_ref = oracle.quantize_rowwise_rhe(W)
        np.testing.assert_array_equal(lin.q.cpu().numpy(), q_ref)
        np.testing.assert_array_equal(lin.scales.cpu().numpy(), s_ref)
    x = torch.randn((4, 64), device=dev).to(torch.bfloat16)
    ref = mj.W8Linear.from_float(torch.from_numpy(W1).to(dev), torch.from_numpy(b1).to(dev))
    assert torch.equal(layers[0].forward(x), ref.forward(x))
