"""Row order of the Gaussian table (mlx3d_amd/splatting/layout.py): the
Morton codes, the permutation and the model / trainer-side reordering,
host-only (CPU tensors)."""

import numpy as np
import torch

from mlx3d_amd.splatting import GaussianModel, spatial_order
from mlx3d_amd.splatting.layout import _spread, morton_codes


def _interleave_brute(x, y, z, bits=10):
    code = 0
    for b in range(bits):
        code |= ((x >> b) & 1) << (3 * b)
        code |= ((y >> b) & 1) << (3 * b + 1)
        code |= ((z >> b) & 1) << (3 * b + 2)
    return code


def test_spread_moves_bit_i_to_3i():
    for b in range(10):
        assert int(_spread(torch.tensor([1 << b]))[0]) == 1 << (3 * b)
    assert int(_spread(torch.tensor([0x3FF]))[0]) == 0x09249249
    # bits above the tenth are dropped
    assert int(_spread(torch.tensor([0x400]))[0]) == 0


def test_codes_match_bitwise_interleaving():
    rng = np.random.default_rng(1)
    q = rng.integers(0, 1024, size=(500, 3))
    # means on the integer grid with the box corners present: quantisation is exact
    m = np.concatenate([q, [[0, 0, 0], [1023, 1023, 1023]]]).astype(np.float64)
    codes = morton_codes(torch.tensor(m)).numpy()
    for i in range(len(m)):
        x, y, z = (int(v) for v in m[i])
        assert codes[i] == _interleave_brute(x, y, z)


def test_order_is_a_stable_sorting_permutation():
    g = torch.Generator().manual_seed(0)
    m = torch.randn(2000, 3, generator=g)
    m[17] = m[5]  # a tie keeps row order
    perm = spatial_order(m)
    assert perm.dtype == torch.int64
    assert sorted(perm.tolist()) == list(range(2000))
    codes = morton_codes(m)[perm]
    assert bool((codes[1:] >= codes[:-1]).all())
    assert perm.tolist().index(5) < perm.tolist().index(17)
    # sorting a sorted table changes nothing
    assert torch.equal(spatial_order(m[perm]), torch.arange(2000))


def test_neighbours_in_space_are_neighbours_in_rows():
    # eight well separated clusters: each one ends up contiguous
    rng = np.random.default_rng(2)
    centres = np.array([[x, y, z] for x in (0, 10) for y in (0, 10) for z in (0, 10)], float)
    lab = rng.integers(0, 8, 4000)
    m = centres[lab] + rng.normal(0, 0.3, (4000, 3))
    perm = spatial_order(torch.tensor(m)).numpy()
    runs = 1 + int((np.diff(lab[perm]) != 0).sum())
    assert runs == 8


def test_degenerate_inputs():
    assert spatial_order(torch.zeros(0, 3)).numel() == 0
    assert spatial_order(torch.ones(5, 3)).tolist() == [0, 1, 2, 3, 4]
    m = torch.tensor([[0.0, 0.0, 0.0], [float("nan"), 1.0, 1.0], [float("inf"), 2.0, 2.0],
                      [1.0, 1.0, 1.0]])
    perm = spatial_order(m)
    assert sorted(perm.tolist()) == [0, 1, 2, 3]
    try:
        spatial_order(torch.zeros(4, 2))
    except ValueError:
        pass
    else:
        raise AssertionError("(N, 2) means accepted")


def test_model_reorder_permutes_every_parameter():
    g = torch.Generator().manual_seed(3)
    n = 300
    params = {"means": torch.randn(n, 3, generator=g), "quats": torch.randn(n, 4, generator=g),
              "scales": torch.randn(n, 3, generator=g), "opacities": torch.randn(n, generator=g),
              "sh_dc": torch.randn(n, 1, 3, generator=g),
              "sh_rest": torch.randn(n, 15, 3, generator=g)}
    before = {k: v.clone() for k, v in params.items()}
    model = GaussianModel(params, sh_degree=3)
    model.requires_grad_(True)
    perm = model.reorder_spatial()
    for k, v in before.items():
        assert torch.equal(model.params[k].detach(), v[perm]), k
        assert model.params[k].requires_grad and model.params[k].is_leaf
    assert torch.equal(perm, spatial_order(before["means"]))
