"""Host-side logic: configuration widths, the seeded generator, workload shapes and the bench /
graft entry-point contracts. No device work."""
import importlib.util
import os

import numpy as np
import pytest

from burn_automata_amd import synthetic as syn
from burn_automata_amd.config import NpaConfig

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
M64 = (1 << 64) - 1


def _stable_uniform_int(seed, stream, pid):
    """stable_particle_uniform (crates/burn_automata/src/rollout/mod.rs:299-308) with Python ints."""
    v = (seed ^ ((stream * 0x9E3779B97F4A7C15) & M64) ^ ((pid * 0xBF58476D1CE4E5B9) & M64)) & M64
    v = ((v ^ (v >> 30)) * 0xBF58476D1CE4E5B9) & M64
    v = ((v ^ (v >> 27)) * 0x94D049BB133111EB) & M64
    v ^= v >> 31
    return (v >> 40) / float(1 << 24)


def test_stable_uniform_matches_integer_restatement():
    ids = np.array([0, 1, 2, 3, 1000, 2 ** 40 + 7, 2 ** 63 + 5], dtype=np.uint64)
    for seed, stream in [(42, 0), (42, 1), (0x5EED5EEDD15CA11C, 3), (M64, 2)]:
        got = syn.stable_uniform(seed, stream, ids)
        want = [_stable_uniform_int(seed, stream, int(i)) for i in ids]
        assert got.tolist() == want
    u = syn.stable_uniform(42, 0, np.arange(200000, dtype=np.uint64))
    assert u.min() >= 0 and u.max() < 1 and abs(u.mean() - 0.5) < 3e-3
    assert np.all(u * (1 << 24) == np.floor(u * (1 << 24)))  # 24-bit lattice


@pytest.mark.parametrize("name,F,O,n,batch", [("c1", 64, 18, 4096, 1), ("c1_dgrad", 66, 18, 4096, 1),
                                             ("c2", 64, 18, 65536, 1), ("c4", 80, 19, 16384, 1)])
def test_workload_shapes(name, F, O, n, batch):
    w = syn.workload(name, particles=None if name != "c2" else 4096)
    m = w["model"]
    assert m.perception_dims() == F and m.update_dims() == O
    n = n if name != "c2" else 4096
    assert w["positions"].shape == (batch * n, 4) and w["positions"].dtype == np.float32
    assert w["states"].shape == (batch * n, m.state_dims)
    assert w["weights"]["w1"].size == m.hidden_dims * F  # row-major w1[H][F]
    assert w["weights"]["w2"].size == O * m.hidden_dims  # w2[O][H]
    assert np.all(w["weights"]["b1"] == 0) and np.abs(w["weights"]["w1"]).max() <= 0.1
    assert abs(float(np.std(w["states"])) - 0.1) < 0.01


def test_c2_decode_configuration():
    w = syn.workload("c2", particles=1024)
    s = w["splat"]
    assert w["decode_every"] == 32 and s.image_size == 512
    assert s.sigma == pytest.approx(0.004 * 511 / 2) and s.pixel_size == pytest.approx(2 / 512)


def test_c5_weights_are_bf16_rounded():
    w = syn.workload("c5", particles=64)
    bits = w["weights"]["w1"].view(np.uint32)
    assert np.all(bits & 0xFFFF == 0) and w["batch"] == 64


def test_model_presets_feature_widths():
    """perception_dims = 2S + S d [+ d] [+ d] (crates/burn_automata/src/config.rs:133-139)."""
    m = NpaConfig.growing_2d().replace(state_dims=16)
    assert m.perception_dims() == 2 * 16 + 16 * 2 + 2 * int(m.density_grad)
    assert m.replace(position_features=True).perception_dims() == m.perception_dims() + 2


def _load(name):
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, f"{name}.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_bench_refuses_more_than_one_gpu(capsys):
    bench = _load("bench")
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err


def test_bench_kernel_work_counts():
    bench = _load("bench")
    m = syn.workload("c1", particles=64)["model"]
    counts = {"candidates": 1000.0, "pairs": 300.0, "targets": 40.0, "target_candidates": 400.0,
              "target_pairs": 120.0}
    work = bench.kernel_work(m, counts, particles=100)
    fl, by = work["mlp"]
    # the MLP runs over the update mask's targets only
    assert fl == 40 * (2 * (64 * 128 + 128 * 18) + 8 + 6 + 48)
    assert by == 40 * (4 * 64 + 4 + 32 + 8 * 16)
    assert work["density"] == (5 * 1000 + 5 * 300 + 100, 100 * 24)
    per_pair = 4 + 1 + 2 * 16 + 7 + 2 + 16 * 5 + 8
    assert work["perceive"][0] == 5 * 400 + per_pair * 120 + 40 * (15 + 128 + 32 + 16 * 29)
    assert work["perceive"][1] == 40 * (16 + 64 + 8 + 256)


def test_graft_entry_points_exist():
    g = _load("__graft_entry__")
    assert callable(g.build) and callable(g.smoke)


def test_raster_camera_look_at():
    """RasterCamera.look_at (bevy's Transform::looking_at + default PerspectiveProjection): the view
    rotation is orthonormal and right-handed, the eye maps to the origin, the target lies on the -z
    axis at its distance, world up projects to +y, and fy = (height / 2) / tan(fov_y / 2)."""
    import math

    import numpy as np

    from burn_automata_amd.config import RasterCamera

    eye, target = np.array([0.6, -0.4, 2.2]), np.array([0.1, 0.2, -0.3])
    cam = RasterCamera.look_at(tuple(eye), tuple(target), width=320, height=240)
    V = np.array(cam.view, np.float64).reshape(4, 4)
    R = V[:3, :3]
    np.testing.assert_allclose(R @ R.T, np.eye(3), atol=1e-12)
    assert abs(np.linalg.det(R) - 1.0) < 1e-12
    np.testing.assert_allclose(V @ np.append(eye, 1.0), [0, 0, 0, 1], atol=1e-12)
    t = V @ np.append(target, 1.0)
    np.testing.assert_allclose(t[:2], 0.0, atol=1e-12)
    assert abs(t[2] + np.linalg.norm(target - eye)) < 1e-12
    up = R @ np.array([0.0, 1.0, 0.0])
    assert up[1] > 0 and abs(up[0]) < 1e-12  # world up stays in the camera's y-z plane, pointing up
    assert abs(cam.fy - 120.0 / math.tan(math.pi / 8)) < 1e-9 and cam.fx == cam.fy
    assert (cam.cx, cam.cy) == (160.0, 120.0)


def test_mean_dx_norm_is_a_serial_f32_mean():
    """rollout/mod.rs:277-282: |dx| over x, y, z only (the fourth lane is padding), summed left to
    right in f32, so a large leading norm swallows the unit norms after it, which a pairwise or
    f64 sum would keep."""
    from burn_automata_amd.rollout import mean_dx_norm
    assert mean_dx_norm(np.zeros((0, 4), np.float32)) == 0.0
    assert mean_dx_norm(np.array([[3, 4, 0, 100], [0, 0, 12, 7]], np.float32)) == 8.5
    dx = np.zeros((5, 4), np.float32)
    dx[:, 0] = [2.0 ** 24, 1, 1, 1, 1]
    assert mean_dx_norm(dx) == float(np.float32(2.0 ** 24) / np.float32(5))
    assert mean_dx_norm(dx) != float(np.float32((2.0 ** 24 + 4) / 5))
