"""Weight files: momijo's checkpoint format, and a binary int8 format for the
per-channel weight path.

momijo's checkpoint (learn/utils/checkpoint.mojo:19-140, checkpoint_fileio.
mojo:86-114) is a JSON header ``{"params":[{"type":"Linear","w":nW,"b":nB},
...]}`` plus one flat Float32 blob holding each layer's weight [OutF, InF]
then its bias, in layer order; the blob is written as ASCII CSV
(learn/utils/tensor_bytes.mojo:40-85; its "binary" wrappers fall back to the
CSV).  ``make_checkpoint`` / ``apply_checkpoint`` / ``pack_csv`` /
``unpack_csv`` reproduce that format.

The int8 file (``save_w8`` / ``load_w8``) has no reference counterpart: the
CSV blob cannot hold int8 weights and their scales, so quantized layers could
not persist.  Layout, little-endian:

    0   b"MJW8", u32 version (1), u32 header bytes H, u32 0
    16  H bytes of UTF-8 JSON: {"layers": [{"name", "out", "in", "rounding",
        "q": [offset, bytes, crc32], "scales": [...], "bias": [...] | null}]}
    ... sections at 256-byte aligned offsets: q int8 [out, in] row-major,
        scales fp32 [out], bias fp32 [out]

Sections are aligned so a memory-mapped file copies straight into HBM; each
carries a CRC-32 that ``load_w8`` verifies.
"""
from __future__ import annotations

import json
import struct
import zlib
from dataclasses import dataclass

import numpy as np

MAGIC = b"MJW8"
VERSION = 1
_ALIGN = 256


# ------------------------------------------------------------ momijo format
def make_checkpoint(layers) -> tuple[str, np.ndarray]:
    """make_checkpoint (learn/utils/checkpoint.mojo:19-100) for a list of
    (weight [OutF, InF], bias [OutF] or empty) Float32 arrays: returns the
    header JSON string and the flat blob."""
    parts, entries = [], []
    for W, b in layers:
        W = np.ascontiguousarray(W, np.float32)
        b = np.ascontiguousarray(b if b is not None else np.zeros(0), np.float32)
        parts += [W.ravel(), b.ravel()]
        entries.append('{"type":"Linear","w":%d,"b":%d}' % (W.size, b.size))
    header = '{"params":[' + ",".join(entries) + "]}"
    blob = np.concatenate(parts) if parts else np.zeros(0, np.float32)
    return header, blob


def apply_checkpoint(shapes, header: str, blob: np.ndarray):
    """apply_checkpoint (learn/utils/checkpoint.mojo:107-140): walks the blob in
    layer order for layers of the given ((OutF, InF), has_bias) shapes; the
    header is not consulted, as in the reference.  Returns [(W, b), ...], or
    None when the blob is too short (the reference would read past it)."""
    del header
    blob = np.asarray(blob, np.float32).ravel()
    out, k = [], 0
    for (out_f, in_f), has_bias in shapes:
        nW, nB = out_f * in_f, out_f if has_bias else 0
        if k + nW + nB > blob.size:
            return None
        W = blob[k:k + nW].reshape(out_f, in_f).copy()
        k += nW
        b = blob[k:k + nB].copy()
        k += nB
        out.append((W, b))
    return out


def pack_csv(x: np.ndarray) -> bytes:
    """pack_f64_to_bytes (learn/utils/tensor_bytes.mojo:40-50): values joined
    by ','.  Each value is written as the shortest decimal that reads back
    to the same Float32 (Mojo's own String(Float32) spelling is not available
    here; any reader that rounds correctly gets identical values back)."""
    x = np.asarray(x, np.float32).ravel()
    return ",".join(np.format_float_positional(v, unique=True, trim="-")
                    if np.isfinite(v) else repr(float(v)) for v in x).encode("ascii")


def unpack_csv(data: bytes) -> np.ndarray:
    """unpack_bytes_to_f64 (learn/utils/tensor_bytes.mojo:53-81): split on
    ',', skip empty fields, a field that does not parse becomes 0.0."""
    vals = []
    for tok in data.decode("utf-8", errors="replace").split(","):
        if not tok:
            continue
        try:
            vals.append(np.float32(float(tok)))
        except ValueError:
            vals.append(np.float32(0.0))
    return np.array(vals, np.float32)


# ------------------------------------------------------------ int8 file
@dataclass
class W8Entry:
    name: str
    q: np.ndarray            # int8 [out, in]
    scales: np.ndarray       # fp32 [out]
    bias: np.ndarray | None  # fp32 [out] or None
    rounding: str = "rhe"


def _pad(n: int) -> int:
    return (n + _ALIGN - 1) // _ALIGN * _ALIGN


def save_w8(path: str, entries) -> None:
    """Writes int8 layers (W8Entry, or objects with q/scales/bias tensors) to
    an MJW8 file."""
    items = []
    for i, e in enumerate(entries):
        q = _host(e.q, np.int8)
        s = _host(e.scales, np.float32)
        b = None if e.bias is None else _host(e.bias, np.float32)
        if q.ndim != 2 or s.shape != (q.shape[0],) or (b is not None and b.shape != s.shape):
            raise ValueError(f"layer {i}: q [out, in], scales [out], bias [out] expected")
        items.append((getattr(e, "name", f"layer{i}"), q, s, b,
                      getattr(e, "rounding", "rhe")))
    # lay out the sections after a header of known size: size the JSON with
    # placeholder offsets first, then fill them in (the width is fixed)
    def header_for(offsets):
        layers = []
        for (name, q, s, b, rnd), (oq, os_, ob) in zip(items, offsets):
            sec = lambda a, o: [o, int(a.nbytes), zlib.crc32(a.tobytes()) & 0xFFFFFFFF]
            layers.append({"name": name, "out": int(q.shape[0]), "in": int(q.shape[1]),
                           "rounding": rnd, "q": sec(q, oq), "scales": sec(s, os_),
                           "bias": None if b is None else sec(b, ob)})
        return json.dumps({"layers": layers}, separators=(",", ":")).encode("utf-8")

    big = 1 << 62
    hdr_len = len(header_for([(big, big, big)] * len(items)))
    pos = _pad(16 + hdr_len)
    offsets = []
    for _, q, s, b, _ in items:
        oq = pos
        pos = _pad(pos + q.nbytes)
        os_ = pos
        pos = _pad(pos + s.nbytes)
        ob = pos if b is not None else 0
        if b is not None:
            pos = _pad(pos + b.nbytes)
        offsets.append((oq, os_, ob))
    hdr = header_for(offsets)
    hdr = hdr + b" " * (hdr_len - len(hdr))  # same width as the placeholder layout
    with open(path, "wb") as f:
        f.write(MAGIC + struct.pack("<III", VERSION, len(hdr), 0))
        f.write(hdr)
        for (_, q, s, b, _), (oq, os_, ob) in zip(items, offsets):
            for a, o in ((q, oq), (s, os_)) + (((b, ob),) if b is not None else ()):
                f.seek(o)
                f.write(a.tobytes())
        f.truncate(pos)


def load_w8(path: str, device=None, verify: bool = True):
    """Reads an MJW8 file.  With a device, returns W8Linear layers whose
    tensors live in its HBM (the sections are memory-mapped and copied);
    without one, W8Entry records of numpy arrays.  Raises ValueError on a bad
    magic, version, bounds or CRC."""
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    if mm.size < 16 or bytes(mm[:4]) != MAGIC:
        raise ValueError(f"{path}: not an MJW8 file")
    version, hlen, _ = struct.unpack("<III", bytes(mm[4:16]))
    if version != VERSION:
        raise ValueError(f"{path}: unsupported version {version}")
    if 16 + hlen > mm.size:
        raise ValueError(f"{path}: truncated header")
    meta = json.loads(bytes(mm[16:16 + hlen]).decode("utf-8"))

    def section(sec, dtype, shape):
        off, nbytes, crc = sec
        if off % _ALIGN or off + nbytes > mm.size or nbytes != int(np.prod(shape)) * np.dtype(dtype).itemsize:
            raise ValueError(f"{path}: section out of bounds or mis-sized")
        raw = mm[off:off + nbytes]
        if verify and (zlib.crc32(raw) & 0xFFFFFFFF) != crc:
            raise ValueError(f"{path}: CRC mismatch")
        return raw.view(dtype).reshape(shape)

    out = []
    for L in meta["layers"]:
        n, k = int(L["out"]), int(L["in"])
        q = section(L["q"], np.int8, (n, k))
        s = section(L["scales"], np.float32, (n,))
        b = None if L["bias"] is None else section(L["bias"], np.float32, (n,))
        if device is None:
            out.append(W8Entry(L["name"], np.array(q), np.array(s),
                               None if b is None else np.array(b), L["rounding"]))
        else:
            import torch
            from .nn import W8Linear
            tdt = {np.dtype(np.int8): torch.int8, np.dtype(np.float32): torch.float32}

            def dev(a):  # file -> pinned staging buffer -> HBM
                t = torch.empty(a.shape, dtype=tdt[a.dtype], pin_memory=True)
                t.numpy()[...] = a
                return t.to(device, non_blocking=True)
            lin = W8Linear(dev(q), dev(s), None if b is None else dev(b))
            torch.cuda.current_stream(device).synchronize()  # staging buffers are freed next
            lin.name, lin.rounding = L["name"], L["rounding"]
            out.append(lin)
    return out


def quantize_checkpoint(header: str, blob: np.ndarray, shapes, path: str, device,
                        rounding: str = "rhe") -> None:
    """momijo fp32 checkpoint -> MJW8 file: each Linear weight is quantized per
    output channel on the device (mj_quantize_rowwise_i8) and written with its
    scales and bias."""
    import torch
    from . import _lib
    from .nn import quantize_rowwise_int8
    layers = apply_checkpoint(shapes, header, blob)
    if layers is None:
        raise ValueError("checkpoint blob is shorter than the layer shapes")
    rule = _lib.ROUND_RHE if rounding == "rhe" else _lib.ROUND_LEGACY
    entries = []
    for i, (W, b) in enumerate(layers):
        q, s = quantize_rowwise_int8(torch.from_numpy(W).to(device), rule)
        entries.append(W8Entry(f"layer{i}", q.cpu().numpy(), s.cpu().numpy(),
                               b if b.size else None, rounding))
    save_w8(path, entries)


def _host(a, dtype) -> np.ndarray:
    if hasattr(a, "detach"):
        a = a.detach().cpu().numpy()
    return np.ascontiguousarray(a, dtype)


__all__ = ["make_checkpoint", "apply_checkpoint", "pack_csv", "unpack_csv", "W8Entry",
           "save_w8", "load_w8", "quantize_checkpoint"]
