"""PLY files: Gaussian checkpoints, point clouds and triangle meshes.

The interface is the reference's (``src/mlx3d/io/ply_io.py:37-271``):
``load_ply(path) -> PlyData`` and ``save_ply(path, verts, faces=None,
normals=None, colors=None, extra=None, binary=True)``, with the same
observable conventions -- uchar colours scaled to [0, 1] on load (values
above 1 mean a 0-255 range), an ``alpha`` property consumed with the colours,
every other vertex property returned in ``extra``, polygons fan-triangulated.

The implementation is a small schema model of the PLY header: each element
becomes a numpy record type, so a binary element without list properties is
one zero-copy ``frombuffer`` view, a triangle-only face list is a second
record view (count + three indices), and only polygons of mixed size take a
per-polygon walk.  ASCII bodies are read as one token stream.  Writing goes
the other way: the columns are gathered into one record array and written
with a single ``tobytes``; ASCII floats use 9 significant digits, enough to
round-trip every float32 exactly.  Values come back as CPU torch tensors;
``GaussianModel.load_ply`` moves a checkpoint's whole vertex table to the GPU
in one copy via :func:`read_ply_vertices`.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field

import numpy as np
import torch

__all__ = ["PlyData", "load_ply", "read_ply_vertices", "save_ply"]

# PLY scalar type names (both spellings of the format) -> numpy type codes
_TYPES = {}
for _codes, _names in (("i1", ("char", "int8")), ("u1", ("uchar", "uint8")),
                       ("i2", ("short", "int16")), ("u2", ("ushort", "uint16")),
                       ("i4", ("int", "int32")), ("u4", ("uint", "uint32")),
                       ("f4", ("float", "float32")), ("f8", ("double", "float64"))):
    for _n in _names:
        _TYPES[_n] = np.dtype("<" + _codes)

_HEADER_END = b"end_header"
_ENCODINGS = ("ascii", "binary_little_endian")


@dataclass
class PlyData:
    """What :func:`load_ply` returns (ply_io.py:37-52): ``verts`` (V, 3),
    ``faces`` (F, 3) int32 or None, ``normals`` / ``colors`` (V, 3) or None
    (colours in [0, 1]), ``extra``: every other vertex property, (V,) each."""

    verts: torch.Tensor
    faces: torch.Tensor | None = None
    normals: torch.Tensor | None = None
    colors: torch.Tensor | None = None
    extra: dict[str, torch.Tensor] = field(default_factory=dict)


@dataclass(frozen=True)
class _Prop:
    name: str
    dtype: np.dtype
    length_dtype: np.dtype | None = None  # set for list properties


@dataclass
class _Element:
    name: str
    size: int
    props: list[_Prop] = field(default_factory=list)

    @property
    def fixed(self) -> bool:
        return all(p.length_dtype is None for p in self.props)

    def record(self) -> np.dtype:
        return np.dtype([(p.name, p.dtype) for p in self.props])


def _schema(buf, path: str):
    """(encoding, elements, body offset) of a PLY header."""
    stop = buf.find(_HEADER_END)
    if stop < 0:
        raise ValueError(f"{path!r}: no 'end_header' line, so not a readable PLY file.")
    body = buf.find(b"\n", stop)
    body = len(buf) if body < 0 else body + 1
    lines = bytes(buf[:stop]).decode("ascii", errors="replace").splitlines()
    if not lines or lines[0].strip() != "ply":
        raise ValueError(f"{path!r} is not a PLY file (missing the 'ply' magic line).")
    encoding = None
    elements: list[_Element] = []
    for raw in lines[1:]:
        tok = raw.split()
        if not tok or tok[0] in ("comment", "obj_info"):
            continue
        kind = tok[0]
        if kind == "format":
            encoding = tok[1] if len(tok) > 1 else None
        elif kind == "element":
            elements.append(_Element(tok[1], int(tok[2])))
        elif kind == "property":
            if not elements:
                raise ValueError(f"{path!r}: a property line comes before any element line.")
            try:
                if tok[1] == "list":
                    prop = _Prop(tok[4], _TYPES[tok[3]], _TYPES[tok[2]])
                else:
                    prop = _Prop(tok[2], _TYPES[tok[1]])
            except (KeyError, IndexError) as e:
                raise ValueError(f"{path!r}: cannot read the property line {raw!r}.") from e
            elements[-1].props.append(prop)
    if encoding not in _ENCODINGS:
        raise ValueError(f"Unsupported PLY format {encoding!r} in {path!r} "
                         f"(supported: {', '.join(_ENCODINGS)}).")
    return encoding, elements, body


def _fan(polygons) -> np.ndarray:
    """Fan triangulation (p0, p_k, p_k+1), polygon by polygon, as int32 (T, 3)."""
    tris = [(p[0], p[k], p[k + 1]) for p in polygons for k in range(1, len(p) - 1)]
    return np.asarray(tris, dtype=np.int32).reshape(-1, 3)


def _binary_list_element(buf, off: int, el: _Element):
    """(triangles, end offset) of a binary element with one list property."""
    if len(el.props) != 1:
        raise ValueError(f"element {el.name!r}: only a single list property is supported")
    prop = el.props[0]
    if el.size == 0:
        return np.zeros((0, 3), np.int32), off
    first = int(np.frombuffer(buf, prop.length_dtype, 1, off)[0])
    rec = np.dtype([("n", prop.length_dtype), ("i", prop.dtype, (first,))])
    if off + rec.itemsize * el.size <= len(buf):
        view = np.frombuffer(buf, rec, el.size, off)
        if (view["n"] == first).all():  # every polygon has the first one's size
            idx = view["i"].reshape(el.size, first).astype(np.int64)
            if first == 3:
                return idx.astype(np.int32), off + rec.itemsize * el.size
            return _fan(idx.tolist()), off + rec.itemsize * el.size
    polys = []
    for _ in range(el.size):  # mixed polygon sizes: walk record by record
        k = int(np.frombuffer(buf, prop.length_dtype, 1, off)[0])
        off += prop.length_dtype.itemsize
        polys.append(np.frombuffer(buf, prop.dtype, k, off).tolist())
        off += prop.dtype.itemsize * k
    return _fan(polys), off


def _parse_body(buf, encoding: str, elements, off: int) -> dict:
    """{element name: {property: (count,) array}}; an element with a list
    property gives {"faces": (T, 3) int32} instead."""
    out: dict = {}
    tokens = bytes(buf[off:]).split() if encoding == "ascii" else None
    pos = 0
    for el in elements:
        if el.fixed:
            if tokens is not None:
                width = len(el.props)
                flat = np.asarray(tokens[pos:pos + width * el.size], dtype=np.float64)
                pos += width * el.size
                table = flat.reshape(el.size, width)
                out[el.name] = {p.name: table[:, j].astype(p.dtype) for j, p in enumerate(el.props)}
            else:
                rec = el.record()
                arr = np.frombuffer(buf, rec, el.size, off)
                off += rec.itemsize * el.size
                out[el.name] = {p.name: arr[p.name] for p in el.props}
            continue
        if tokens is not None:
            polys = []
            for _ in range(el.size):
                k = int(tokens[pos])
                polys.append([int(t) for t in tokens[pos + 1:pos + 1 + k]])
                pos += 1 + k
            tris = _fan(polys)
        else:
            tris, off = _binary_list_element(buf, off, el)
        out[el.name] = {"faces": tris}
    return out


def _slurp(path: str):
    """The file's bytes in a writable buffer (arrays viewing it can back
    torch tensors without a copy)."""
    buf = bytearray(os.path.getsize(path))
    with open(path, "rb") as f:
        f.readinto(buf)
    return buf


def load_ply(path: str) -> PlyData:
    """Read an ascii or binary_little_endian PLY file (ply_io.py:56-182)."""
    buf = _slurp(path)
    encoding, elements, body = _schema(buf, path)
    parsed = _parse_body(buf, encoding, elements, body)
    vertex = parsed.get("vertex")
    if vertex is None:
        raise ValueError(f"{path!r} has no vertex element.")
    missing = [a for a in "xyz" if a not in vertex]
    if missing:
        raise ValueError(f"{path!r}: the vertex element lacks the {', '.join(missing)} "
                         "coordinate(s).")

    def f32(cols):
        return torch.from_numpy(np.stack([np.asarray(vertex[c], np.float32) for c in cols], -1))

    taken = {"x", "y", "z"}
    normals = colors = None
    if {"nx", "ny", "nz"} <= vertex.keys():
        normals = f32(("nx", "ny", "nz"))
        taken |= {"nx", "ny", "nz"}
    if {"red", "green", "blue"} <= vertex.keys():
        colors = f32(("red", "green", "blue"))
        if colors.numel() and float(colors.max()) > 1.0:  # stored as 0..255
            colors = colors / 255.0
        taken |= {"red", "green", "blue", "alpha"}
    extra = {k: torch.from_numpy(np.ascontiguousarray(v, np.float32))
             for k, v in vertex.items() if k not in taken}
    faces = None
    face = parsed.get("face")
    if face is not None and face["faces"].size:
        faces = torch.from_numpy(face["faces"])
    return PlyData(verts=f32(("x", "y", "z")), faces=faces, normals=normals, colors=colors,
                   extra=extra)


def read_ply_vertices(path: str) -> tuple[list[str], np.ndarray]:
    """(property names, (V, P) float32 table) of a binary little-endian file
    whose vertex properties are all float32 (a 3DGS checkpoint): a zero-copy
    view of the file's bytes, columns in file order.  Raises ValueError for
    any other file (``GaussianModel.load_ply`` then reads it generically)."""
    buf = _slurp(path)
    encoding, elements, off = _schema(buf, path)
    for el in elements:
        if el.name == "vertex":
            if encoding != "binary_little_endian" or not el.fixed or any(
                    p.dtype != np.dtype("<f4") for p in el.props):
                raise ValueError("the vertex element is not an all-float32 binary table")
            table = np.frombuffer(buf, np.dtype("<f4"), el.size * len(el.props), off)
            return [p.name for p in el.props], table.reshape(el.size, len(el.props))
        if not el.fixed:
            raise ValueError("a list element precedes the vertex element")
        off += el.record().itemsize * el.size
    raise ValueError(f"{path!r} has no vertex element.")


def _host(a, dtype, shape=None) -> np.ndarray:
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu().numpy()
    a = np.ascontiguousarray(a, dtype=dtype)
    return a.reshape(shape) if shape is not None else a


def save_ply(path: str, verts, faces=None, normals=None, colors=None, extra=None,
             binary: bool = True) -> None:
    """Write points or a triangle mesh (ply_io.py:185-271): float32 x y z,
    optional float32 normals, colours in [0, 1] stored as uchar red green
    blue, ``extra`` properties as float32 in insertion order, faces as
    ``list uchar int vertex_indices`` triangles."""
    v = _host(verts, np.float32, (-1, 3))
    count = v.shape[0]
    columns: list[tuple[str, np.dtype, np.ndarray]] = [
        (a, np.dtype("<f4"), v[:, j]) for j, a in enumerate("xyz")]
    if normals is not None:
        nrm = _host(normals, np.float32, (count, 3))
        columns += [(a, np.dtype("<f4"), nrm[:, j]) for j, a in enumerate(("nx", "ny", "nz"))]
    if colors is not None:
        rgb = np.clip(_host(colors, np.float32, (count, 3)) * 255.0, 0, 255).astype(np.uint8)
        columns += [(a, np.dtype("u1"), rgb[:, j]) for j, a in enumerate(("red", "green", "blue"))]
    for name, vals in (extra or {}).items():
        columns.append((name, np.dtype("<f4"), _host(vals, np.float32, (count,))))
    tris = None if faces is None else _host(faces, np.int64, (-1, 3))

    type_name = {np.dtype("<f4"): "float", np.dtype("u1"): "uchar"}
    lines = ["ply", f"format {'binary_little_endian' if binary else 'ascii'} 1.0",
             f"element vertex {count}"]
    lines += [f"property {type_name[dt]} {name}" for name, dt, _ in columns]
    if tris is not None:
        lines += [f"element face {tris.shape[0]}", "property list uchar int vertex_indices"]
    lines.append("end_header")
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "wb") as out:
        out.write(("\n".join(lines) + "\n").encode("ascii"))
        if binary:
            table = np.empty(count, dtype=[(name, dt) for name, dt, _ in columns])
            for name, _, vals in columns:
                table[name] = vals
            out.write(table.tobytes())
            if tris is not None:
                frec = np.empty(tris.shape[0], dtype=[("n", "u1"), ("i", "<i4", (3,))])
                frec["n"] = 3
                frec["i"] = tris
                out.write(frec.tobytes())
            return
        # ascii: one formatted line per record (floats with 9 significant
        # digits, which round-trips float32)
        fmts = ["%d" if dt.kind == "u" else "%.9g" for _, dt, _ in columns]
        line_fmt = " ".join(fmts) + "\n"
        cols = [vals.astype(np.float64) if dt.kind == "f" else vals.astype(np.int64)
                for _, dt, vals in columns]
        out.write("".join(line_fmt % tuple(c[i] for c in cols) for i in range(count))
                  .encode("ascii"))
        if tris is not None:
            out.write("".join(f"3 {a} {b} {c}\n" for a, b, c in tris.tolist()).encode("ascii"))
