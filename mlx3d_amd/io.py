"""PLY reading and writing (``src/mlx3d/io/ply_io.py``) for Gaussian
checkpoints and point clouds.

``load_ply`` accepts ``ascii`` and ``binary_little_endian`` files with
scalar vertex properties of any PLY type and one list property per face
element (polygons are fan-triangulated); ``save_ply`` writes float32
positions / normals / extra properties, uchar colours and int32 triangle
lists, binary or ascii.  Values come back as CPU torch tensors; Gaussian
checkpoints go to the GPU through ``GaussianModel.load_ply``, which moves the
whole vertex table in one host-to-device copy.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field

import numpy as np
import torch

__all__ = ["PlyData", "load_ply", "read_ply_vertices", "save_ply"]

# ply_io.py:17-34
_PLY_TO_NP = {
    "char": "i1", "int8": "i1", "uchar": "u1", "uint8": "u1",
    "short": "i2", "int16": "i2", "ushort": "u2", "uint16": "u2",
    "int": "i4", "int32": "i4", "uint": "u4", "uint32": "u4",
    "float": "f4", "float32": "f4", "double": "f8", "float64": "f8",
}


@dataclass
class PlyData:
    """Result of :func:`load_ply` (ply_io.py:37-52): ``verts`` (V, 3),
    ``faces`` (F, 3) or None, ``normals`` / ``colors`` (V, 3) or None
    (colours in [0, 1]), ``extra``: every other vertex property, (V,) each."""

    verts: torch.Tensor
    faces: torch.Tensor | None = None
    normals: torch.Tensor | None = None
    colors: torch.Tensor | None = None
    extra: dict[str, torch.Tensor] = field(default_factory=dict)


def _parse_header(data: bytes, path: str):
    end = data.find(b"end_header\n")
    if end < 0:
        raise ValueError(f"{path!r} is not a valid PLY file (no end_header).")
    lines = data[:end].decode("ascii", errors="replace").splitlines()
    if not lines or lines[0].strip() != "ply":
        raise ValueError(f"{path!r} is not a PLY file.")
    fmt = None
    elements: list[tuple[str, int, list]] = []
    for line in lines[1:]:
        parts = line.strip().split()
        if not parts or parts[0] in ("comment", "obj_info"):
            continue
        if parts[0] == "format":
            fmt = parts[1]
        elif parts[0] == "element":
            elements.append((parts[1], int(parts[2]), []))
        elif parts[0] == "property":
            if not elements:
                raise ValueError("property before element in PLY header.")
            if parts[1] == "list":
                elements[-1][2].append(("__list__", parts[4], _PLY_TO_NP[parts[2]],
                                        _PLY_TO_NP[parts[3]]))
            else:
                elements[-1][2].append((parts[2], _PLY_TO_NP[parts[1]]))
    if fmt not in ("ascii", "binary_little_endian"):
        raise ValueError(f"Unsupported PLY format {fmt!r}.")
    return fmt, elements, end + len(b"end_header\n")


def _read_elements(data: bytes, fmt: str, elements, body_off: int):
    """{element: {property: array}}; list elements give {'__faces__': (F, 3)}."""
    parsed: dict[str, dict[str, np.ndarray]] = {}
    off = body_off
    rows = data[body_off:].decode("ascii", errors="replace").splitlines() \
        if fmt == "ascii" else None
    row = 0
    for name, count, props in elements:
        lists = [p for p in props if p[0] == "__list__"]
        if not lists:
            dt = np.dtype([(p[0], "<" + p[1]) for p in props])
            if fmt == "ascii":
                vals = np.array([[float(x) for x in rows[row + i].split()[:len(props)]]
                                 for i in range(count)], dtype=np.float64)
                row += count
                arr = np.empty(count, dt)
                for j, p in enumerate(props):
                    arr[p[0]] = vals[:, j] if count else vals.reshape(0)
            else:
                arr = np.frombuffer(data, dtype=dt, count=count, offset=off)
                off += dt.itemsize * count
            parsed[name] = {p[0]: arr[p[0]] for p in props}
            continue
        # one list property (vertex_indices): fan-triangulate polygons
        polys = []
        if fmt == "ascii":
            for i in range(count):
                vals = rows[row + i].split()
                n = int(vals[0])
                polys.append([int(x) for x in vals[1:1 + n]])
            row += count
        else:
            lp = lists[0]
            cdt, idt = np.dtype("<" + lp[2]), np.dtype("<" + lp[3])
            for _ in range(count):
                n = int(np.frombuffer(data, dtype=cdt, count=1, offset=off)[0])
                off += cdt.itemsize
                polys.append(np.frombuffer(data, dtype=idt, count=n, offset=off).tolist())
                off += idt.itemsize * n
        tris = [[p[0], p[i], p[i + 1]] for p in polys for i in range(1, len(p) - 1)]
        parsed[name] = {"__faces__": np.asarray(tris, dtype=np.int32).reshape(-1, 3)}
    return parsed


def _read(path: str):
    # a writable buffer: arrays viewing it can back torch tensors directly
    data = bytearray(os.path.getsize(path))
    with open(path, "rb") as f:
        f.readinto(data)
    fmt, elements, body = _parse_header(data, path)
    return data, fmt, elements, body


def load_ply(path: str) -> PlyData:
    """Load a PLY file (ply_io.py:56-182)."""
    data, fmt, elements, body = _read(path)
    parsed = _read_elements(data, fmt, elements, body)
    if "vertex" not in parsed:
        raise ValueError(f"No vertex element in {path!r}.")
    vp = parsed["vertex"]
    for axis in ("x", "y", "z"):
        if axis not in vp:
            raise ValueError(f"Vertex element missing {axis!r} property.")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))  # noqa: E731
    verts = np.stack([vp["x"], vp["y"], vp["z"]], axis=-1)
    used = {"x", "y", "z"}
    normals = None
    if all(k in vp for k in ("nx", "ny", "nz")):
        normals = t(np.stack([vp["nx"], vp["ny"], vp["nz"]], axis=-1))
        used |= {"nx", "ny", "nz"}
    colors = None
    if all(k in vp for k in ("red", "green", "blue")):
        rgb = np.stack([vp["red"], vp["green"], vp["blue"]], axis=-1).astype(np.float32)
        if rgb.size and rgb.max() > 1.0:
            rgb = rgb / 255.0
        colors = t(rgb)
        used |= {"red", "green", "blue", "alpha"}
    extra = {k: t(v) for k, v in vp.items() if k not in used}
    faces = None
    if "face" in parsed and parsed["face"]["__faces__"].size > 0:
        faces = torch.from_numpy(parsed["face"]["__faces__"])
    return PlyData(verts=t(verts), faces=faces, normals=normals, colors=colors, extra=extra)


def read_ply_vertices(path: str) -> tuple[list[str], np.ndarray]:
    """(property names, (V, P) float32 table) for a binary little-endian
    file whose vertex properties are all float32 (the 3DGS checkpoint case):
    a zero-copy view of the file's bytes, in file order."""
    data, fmt, elements, body = _read(path)
    off = body
    for name, count, props in elements:
        if name == "vertex":
            if fmt != "binary_little_endian" or any(p[0] == "__list__" or p[1] != "f4"
                                                    for p in props):
                raise ValueError("not an all-float32 binary vertex table")
            arr = np.frombuffer(data, dtype="<f4", count=count * len(props), offset=off)
            return [p[0] for p in props], arr.reshape(count, len(props))
        if any(p[0] == "__list__" for p in props):
            raise ValueError("list element before the vertex element")
        off += np.dtype([(p[0], "<" + p[1]) for p in props]).itemsize * count
    raise ValueError(f"No vertex element in {path!r}.")


def _np32(a, shape=None):
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a.reshape(shape) if shape is not None else a


def save_ply(path: str, verts, faces=None, normals=None, colors=None, extra=None,
             binary: bool = True) -> None:
    """Save points / a triangle mesh (ply_io.py:185-271).  ``colors`` in
    [0, 1] are stored as uchar; ``extra`` properties as float32 in
    insertion order."""
    v = _np32(verts)
    n = _np32(normals) if normals is not None else None
    c = (np.clip(_np32(colors) * 255.0, 0, 255).astype(np.uint8)
         if colors is not None else None)
    ex = {k: _np32(a, (len(v),)) for k, a in (extra or {}).items()}
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    fmt = "binary_little_endian" if binary else "ascii"
    header = ["ply", f"format {fmt} 1.0", f"element vertex {len(v)}"]
    header += [f"property float {a}" for a in ("x", "y", "z")]
    if n is not None:
        header += [f"property float n{a}" for a in ("x", "y", "z")]
    if c is not None:
        header += [f"property uchar {a}" for a in ("red", "green", "blue")]
    header += [f"property float {k}" for k in ex]
    if faces is not None:
        header += [f"element face {len(faces)}", "property list uchar int vertex_indices"]
    header.append("end_header")
    with open(path, "wb") as out:
        out.write(("\n".join(header) + "\n").encode("ascii"))
        if binary:
            fields = [("xyz", "<f4", (3,))]
            if n is not None:
                fields.append(("n", "<f4", (3,)))
            if c is not None:
                fields.append(("rgb", "u1", (3,)))
            fields += [(k, "<f4") for k in ex]
            rec = np.empty(len(v), dtype=np.dtype(fields))
            rec["xyz"] = v
            if n is not None:
                rec["n"] = n
            if c is not None:
                rec["rgb"] = c
            for k, a in ex.items():
                rec[k] = a
            out.write(rec.tobytes())
            if faces is not None:
                f = np.asarray(faces.cpu() if isinstance(faces, torch.Tensor) else faces,
                               dtype=np.int32).reshape(-1, 3)
                frec = np.empty(len(f), dtype=np.dtype([("n", "u1"), ("idx", "<i4", (3,))]))
                frec["n"] = 3
                frec["idx"] = f
                out.write(frec.tobytes())
        else:
            for i in range(len(v)):
                row = [f"{x:.8f}" for x in v[i]]
                if n is not None:
                    row += [f"{x:.8f}" for x in n[i]]
                if c is not None:
                    row += [str(int(x)) for x in c[i]]
                row += [f"{ex[k][i]:.8f}" for k in ex]
                out.write((" ".join(row) + "\n").encode("ascii"))
            if faces is not None:
                f = np.asarray(faces.cpu() if isinstance(faces, torch.Tensor) else faces,
                               dtype=np.int64).reshape(-1, 3)
                for tri in f:
                    out.write(f"3 {tri[0]} {tri[1]} {tri[2]}\n".encode("ascii"))
