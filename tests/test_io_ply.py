"""PLY checkpoints and point clouds (io/ply_io.py, model.py:338-392).

The reference's own I/O tests (test_io.py:343-371, test_splatting.py:545-555)
restated on torch tensors, plus a byte-level known answer: the 3DGS vertex
record built field by field with ``struct`` from the layout definition
(x y z nx ny nz f_dc_0..2 f_rest_* opacity scale_0..2 rot_0..3, f_rest
channel-major) must equal the file GaussianModel.save_ply writes.
"""

from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from mlx3d_amd.io import load_ply, read_ply_vertices, save_ply
from mlx3d_amd.splatting import GaussianModel


def _cube():
    v = torch.tensor([[x, y, z] for x in (0.0, 1.0) for y in (0.0, 1.0) for z in (0.0, 1.0)])
    f = torch.tensor([[0, 1, 3], [0, 3, 2], [4, 6, 7], [4, 7, 5], [0, 4, 5], [0, 5, 1],
                      [2, 3, 7], [2, 7, 6], [0, 2, 6], [0, 6, 4], [1, 5, 7], [1, 7, 3]],
                     dtype=torch.int32)
    return v, f


@pytest.mark.parametrize("binary", [True, False])
def test_ply_roundtrip_mesh(tmp_path, binary):
    verts, faces = _cube()
    p = str(tmp_path / f"cube_{binary}.ply")
    save_ply(p, verts, faces=faces, binary=binary)
    data = load_ply(p)
    torch.testing.assert_close(data.verts, verts)
    assert data.faces.tolist() == faces.tolist()


@pytest.mark.parametrize("binary", [True, False])
def test_ply_pointcloud_with_attrs(tmp_path, binary):
    g = torch.Generator().manual_seed(0)
    pts = torch.randn((50, 3), generator=g)
    normals = torch.randn((50, 3), generator=g)
    colors = torch.rand((50, 3), generator=g)
    extra = {"opacity": torch.randn(50, generator=g), "scale_0": torch.randn(50, generator=g)}
    p = str(tmp_path / f"pc_{binary}.ply")
    save_ply(p, pts, normals=normals, colors=colors, extra=extra, binary=binary)
    data = load_ply(p)
    torch.testing.assert_close(data.verts, pts, atol=1e-5, rtol=0)
    torch.testing.assert_close(data.normals, normals, atol=1e-5, rtol=0)
    torch.testing.assert_close(data.colors, colors, atol=1.0 / 255.0 + 1e-6, rtol=0)
    assert data.faces is None
    assert set(data.extra) == {"opacity", "scale_0"}
    torch.testing.assert_close(data.extra["opacity"], extra["opacity"], atol=1e-5, rtol=0)


def test_ply_quads_fan_triangulated_and_types(tmp_path):
    body = ("ply\nformat ascii 1.0\ncomment hand-made\nelement vertex 5\n"
            "property double x\nproperty double y\nproperty double z\nproperty uchar red\n"
            "property uchar green\nproperty uchar blue\nelement face 2\n"
            "property list uchar int vertex_indices\nend_header\n"
            "0 0 0 255 0 0\n1 0 0 0 255 0\n1 1 0 0 0 255\n0 1 0 255 255 255\n2 2 2 0 0 0\n"
            "4 0 1 2 3\n3 1 4 2\n")
    p = tmp_path / "quad.ply"
    p.write_bytes(body.encode())
    d = load_ply(str(p))
    assert d.faces.tolist() == [[0, 1, 2], [0, 2, 3], [1, 4, 2]]
    torch.testing.assert_close(d.colors[0], torch.tensor([1.0, 0.0, 0.0]))
    assert d.extra == {}


def test_ply_errors(tmp_path):
    p = tmp_path / "bad.ply"
    p.write_bytes(b"ply\nformat ascii 1.0\nelement vertex 0\n")
    with pytest.raises(ValueError, match="end_header"):
        load_ply(str(p))
    p.write_bytes(b"plx\nend_header\n")
    with pytest.raises(ValueError, match="not a PLY"):
        load_ply(str(p))
    p.write_bytes(b"ply\nformat binary_big_endian 1.0\nelement vertex 0\nend_header\n")
    with pytest.raises(ValueError, match="Unsupported"):
        load_ply(str(p))


def _model(n=20, degree=2, seed=0):
    g = torch.Generator().manual_seed(seed)
    K = (degree + 1) ** 2
    params = {"means": torch.randn((n, 3), generator=g),
              "scales": torch.randn((n, 3), generator=g) - 3.0,
              "quats": torch.randn((n, 4), generator=g),
              "opacities": torch.randn(n, generator=g),
              "sh_dc": torch.randn((n, 1, 3), generator=g),
              "sh_rest": torch.randn((n, K - 1, 3), generator=g) * 0.1}
    return GaussianModel(params, sh_degree=degree)


def test_model_ply_roundtrip(tmp_path):
    model = _model()
    p = str(tmp_path / "ckpt.ply")
    model.save_ply(p)
    loaded = GaussianModel.load_ply(p, device="cpu")
    assert loaded.sh_degree == 2 and loaded.active_sh_degree == 2
    for k in model.params:
        assert torch.equal(loaded.params[k], model.params[k]), k


def test_model_ply_known_bytes(tmp_path):
    """The file equals the 3DGS record packed field by field."""
    model = _model(n=3, degree=1, seed=1)
    p = tmp_path / "ckpt.ply"
    model.save_ply(str(p))
    P = model.params
    props = (["x", "y", "z", "nx", "ny", "nz", "f_dc_0", "f_dc_1", "f_dc_2"]
             + [f"f_rest_{i}" for i in range(9)] + ["opacity", "scale_0", "scale_1", "scale_2",
                                                    "rot_0", "rot_1", "rot_2", "rot_3"])
    head = "ply\nformat binary_little_endian 1.0\nelement vertex 3\n"
    head += "".join(f"property float {k}\n" for k in props) + "end_header\n"
    rec = b""
    for i in range(3):
        vals = list(P["means"][i].tolist()) + [0.0, 0.0, 0.0] + list(P["sh_dc"][i, 0].tolist())
        for ch in range(3):  # channel-major: all coefficients of R, then G, then B
            vals += [P["sh_rest"][i, k, ch].item() for k in range(3)]
        vals += [P["opacities"][i].item()] + P["scales"][i].tolist() + P["quats"][i].tolist()
        rec += struct.pack("<26f", *vals)
    assert p.read_bytes() == head.encode() + rec
    # the generic writer with the same properties writes the same bytes
    n = 3
    rest = P["sh_rest"].transpose(1, 2).reshape(n, -1)
    extra = {f"f_dc_{c}": P["sh_dc"][:, 0, c] for c in range(3)}
    extra.update({f"f_rest_{i}": rest[:, i] for i in range(rest.shape[1])})
    extra["opacity"] = P["opacities"]
    extra.update({f"scale_{i}": P["scales"][:, i] for i in range(3)})
    extra.update({f"rot_{i}": P["quats"][:, i] for i in range(4)})
    q = tmp_path / "generic.ply"
    save_ply(str(q), P["means"], normals=torch.zeros((n, 3)), extra=extra)
    assert q.read_bytes() == p.read_bytes()


def test_model_ply_degree_inference_and_generic_path(tmp_path):
    m0 = _model(n=7, degree=0)
    p = str(tmp_path / "d0.ply")
    m0.save_ply(p)
    l0 = GaussianModel.load_ply(p, sh_degree=3, device="cpu")
    assert l0.sh_degree == 0 and l0.params["sh_rest"].shape == (7, 0, 3)
    m1 = _model(n=7, degree=1)
    names, table = read_ply_vertices(str(tmp_path / "d0.ply"))
    assert table.shape == (7, len(names))
    # an ascii checkpoint takes the generic reader and gives the same table
    a = str(tmp_path / "d1_ascii.ply")
    n = 7
    P = m1.params
    rest = P["sh_rest"].transpose(1, 2).reshape(n, -1)
    extra = {f"f_dc_{c}": P["sh_dc"][:, 0, c] for c in range(3)}
    extra.update({f"f_rest_{i}": rest[:, i] for i in range(rest.shape[1])})
    extra["opacity"] = P["opacities"]
    extra.update({f"scale_{i}": P["scales"][:, i] for i in range(3)})
    extra.update({f"rot_{i}": P["quats"][:, i] for i in range(4)})
    save_ply(a, P["means"], normals=torch.zeros((n, 3)), extra=extra, binary=False)
    la = GaussianModel.load_ply(a, device="cpu")
    assert la.sh_degree == 1
    for k in P:
        torch.testing.assert_close(la.params[k], P[k], atol=1e-7, rtol=1e-7)


def test_ply_binary_polygons_and_alpha(tmp_path):
    """Binary faces: uniform quads (one record view) and mixed sizes (the
    per-polygon walk) triangulate as fans; an alpha property is consumed with
    the colours; ushort/double properties load as float32 extras."""
    head = ("ply\nformat binary_little_endian 1.0\nelement vertex 4\n"
            "property double x\nproperty double y\nproperty double z\n"
            "property uchar red\nproperty uchar green\nproperty uchar blue\nproperty uchar alpha\n"
            "property ushort label\nelement face {nf}\nproperty list uchar uint vertex_indices\n"
            "end_header\n")
    verts = b"".join(struct.pack("<3d4BH", x, y, 0.0, 255, 128, 0, 255, i)
                     for i, (x, y) in enumerate([(0, 0), (1, 0), (1, 1), (0, 1)]))
    quads = struct.pack("<B4I", 4, 0, 1, 2, 3) + struct.pack("<B4I", 4, 3, 2, 1, 0)
    mixed = struct.pack("<B3I", 3, 0, 1, 2) + struct.pack("<B4I", 4, 0, 1, 2, 3)
    for name, faces, nf, want in [
            ("quads", quads, 2, [[0, 1, 2], [0, 2, 3], [3, 2, 1], [3, 1, 0]]),
            ("mixed", mixed, 2, [[0, 1, 2], [0, 1, 2], [0, 2, 3]])]:
        p = tmp_path / f"{name}.ply"
        p.write_bytes(head.format(nf=nf).encode() + verts + faces)
        d = load_ply(str(p))
        assert d.faces.tolist() == want, name
        assert d.faces.dtype == torch.int32
        torch.testing.assert_close(d.colors[0], torch.tensor([1.0, 128 / 255, 0.0]))
        assert set(d.extra) == {"label"}
        assert d.extra["label"].tolist() == [0.0, 1.0, 2.0, 3.0]
        assert d.verts.dtype == torch.float32 and d.verts[2].tolist() == [1.0, 1.0, 0.0]


def test_ply_ascii_floats_round_trip_exactly(tmp_path):
    """The ascii writer's 9 significant digits round-trip every float32,
    tiny and huge magnitudes included."""
    vals = np.array([1e-30, -3.4e38, 0.1, 1 / 3, 2.0 ** -126, 123456.789], np.float32)
    pts = torch.from_numpy(np.stack([vals, vals[::-1].copy(), -vals], 1))
    p = str(tmp_path / "exact.ply")
    save_ply(p, pts, extra={"v": torch.from_numpy(vals)}, binary=False)
    d = load_ply(p)
    assert torch.equal(d.verts, pts)
    assert torch.equal(d.extra["v"], torch.from_numpy(vals))
