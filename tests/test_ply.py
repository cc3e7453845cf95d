"""3DGS .ply and cameras.json I/O (src/gaussians.jl:553-592, 839-968; src/cameras.jl:403-522).

The reference's own tests hold no model or camera files, so the formats are pinned by what the
file layouts fix independently of this reader and writer: the byte layout of a binary little
endian PLY with the SIBR property order, files written here by hand (other property orders,
double precision, big endian, ASCII), the original 3DGS f_rest convention (features_rest
(n, h-1, 3) transposed to (n, 3, h-1) and flattened), and the covariance and opacity values of
test/gaussians.jl:85-97.
"""
import json

import numpy as np
import pytest

from tdgs_amd import host, ply

f32 = np.float32


def _random_gaussians(n, degree, seed):
    rng = np.random.default_rng(seed)
    h = (degree + 1) ** 2
    return host.HostGaussians(rng.standard_normal((n, 4)).astype(f32),
                              rng.standard_normal((n, 3)).astype(f32),
                              rng.standard_normal((n, 4)).astype(f32),
                              rng.standard_normal((n, 3, h)).astype(f32))


def _header(path):
    with open(path, "rb") as fh:
        data = fh.read()
    end = data.index(b"end_header\n") + len(b"end_header\n")
    return data[:end].decode("ascii").splitlines(), data[end:]


def _expected_names(h, normals=False):
    names = ["x", "y", "z"] + (["nx", "ny", "nz"] if normals else [])
    names += [f"f_dc_{c}" for c in range(3)] + [f"f_rest_{k}" for k in range(3 * (h - 1))]
    return names + ["opacity", "scale_0", "scale_1", "scale_2", "rot_0", "rot_1", "rot_2", "rot_3"]


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_ply_round_trip_bit_exact(tmp_path, degree):
    g = _random_gaussians(257, degree, degree)
    p = tmp_path / "m.ply"
    ply.save_3dgs_ply(p, g)
    r = ply.read_3dgs_ply(p)
    for a, b in ((g.means_opacity, r.means_opacity), (g.scaling, r.scaling), (g.rotation, r.rotation),
                 (g.sh, r.sh)):
        assert b.dtype == np.float32 and b.shape == a.shape
        np.testing.assert_array_equal(a, b)


def test_ply_byte_layout_sibr_order(tmp_path):
    g = _random_gaussians(5, 3, 7)
    p = tmp_path / "m.ply"
    ply.save_3dgs_ply(p, g)
    lines, body = _header(p)
    assert lines[:3] == ["ply", "format binary_little_endian 1.0", "element vertex 5"]
    assert lines[-1] == "end_header"
    props = [ln.split() for ln in lines[3:-1]]
    assert all(w[:2] == ["property", "float32"] for w in props)
    names = [w[2] for w in props]
    assert names == _expected_names(16) and len(names) == 59
    assert len(body) == 5 * 59 * 4
    rows = np.frombuffer(body, dtype="<f4").reshape(5, 59)
    np.testing.assert_array_equal(rows[:, 0:3], g.means_opacity[:, :3])
    np.testing.assert_array_equal(rows[:, 3:6], g.sh[:, :, 0])
    # f_rest_k = coefficient 1 + k % 15 of channel k // 15 (features_rest transposed, flattened)
    np.testing.assert_array_equal(rows[:, 6:51], g.sh[:, :, 1:].reshape(5, 45))
    np.testing.assert_array_equal(rows[:, 51], g.means_opacity[:, 3])
    np.testing.assert_array_equal(rows[:, 52:55], g.scaling)
    np.testing.assert_array_equal(rows[:, 55:59], g.rotation)


def test_ply_options_normals_padding_float_name(tmp_path):
    g = _random_gaussians(4, 1, 3)
    p = tmp_path / "m.ply"
    ply.save_3dgs_ply(p, g, force_sh_degree_3=True, include_normals=True, use_float_double=True)
    lines, body = _header(p)
    props = [ln.split() for ln in lines[3:-1]]
    assert all(w[1] == "float" for w in props)
    assert [w[2] for w in props] == _expected_names(16, normals=True)
    rows = np.frombuffer(body, dtype="<f4").reshape(4, 62)
    np.testing.assert_array_equal(rows[:, 3:6], 0)
    rest = rows[:, 9:54].reshape(4, 3, 15)
    np.testing.assert_array_equal(rest[:, :, :3], g.sh[:, :, 1:])
    np.testing.assert_array_equal(rest[:, :, 3:], 0)
    r = ply.read_3dgs_ply(p)
    assert r.sh_degree == 3
    np.testing.assert_array_equal(r.sh[:, :, :4], g.sh)
    np.testing.assert_array_equal(r.sh[:, :, 4:], 0)


def _write_foreign_ply(path, cols, fmt, ftype):
    """A PLY written without the module's writer: shuffled property order, any type, any format."""
    n = len(next(iter(cols.values())))
    names = list(cols)
    np_t = {"float": "f4", "double": "f8"}[ftype]
    head = ["ply", f"format {fmt} 1.0", "comment written by hand", "element vertex %d" % n]
    head += [f"property {ftype} {k}" for k in names]
    head += ["element face 0", "property list uchar int vertex_indices", "end_header"]
    with open(path, "wb") as fh:
        fh.write(("\n".join(head) + "\n").encode("ascii"))
        if fmt == "ascii":
            for i in range(n):
                fh.write((" ".join(repr(float(cols[k][i])) for k in names) + "\n").encode("ascii"))
        else:
            order = "<" if fmt == "binary_little_endian" else ">"
            dt = np.dtype([(k, order + np_t) for k in names])
            rec = np.empty(n, dtype=dt)
            for k in names:
                rec[k] = cols[k]
            fh.write(rec.tobytes())


@pytest.mark.parametrize("fmt,ftype", [("binary_little_endian", "double"), ("binary_big_endian", "float"),
                                       ("ascii", "float")])
def test_ply_reads_other_orders_types_formats(tmp_path, fmt, ftype):
    g = _random_gaussians(9, 2, 11)
    cols = {f"f_rest_{k}": g.sh[:, k // 8, 1 + k % 8] for k in reversed(range(24))}
    cols.update({"rot_3": g.rotation[:, 3], "opacity": g.means_opacity[:, 3], "z": g.means_opacity[:, 2]})
    cols.update({f"scale_{i}": g.scaling[:, i] for i in range(3)})
    cols.update({"y": g.means_opacity[:, 1], "x": g.means_opacity[:, 0]})
    cols.update({f"rot_{i}": g.rotation[:, i] for i in range(3)})
    cols.update({f"f_dc_{c}": g.sh[:, c, 0] for c in range(3)})
    cols["red"] = np.arange(9, dtype=f32)  # extra properties are ignored
    p = tmp_path / "foreign.ply"
    _write_foreign_ply(p, cols, fmt, ftype)
    r = ply.read_3dgs_ply(p)
    np.testing.assert_array_equal(r.means_opacity, g.means_opacity)
    np.testing.assert_array_equal(r.scaling, g.scaling)
    np.testing.assert_array_equal(r.rotation, g.rotation)
    np.testing.assert_array_equal(r.sh, g.sh)


def test_ply_rejects_malformed(tmp_path):
    g = _random_gaussians(3, 0, 1)
    cols = {"x": g.means_opacity[:, 0], "y": g.means_opacity[:, 1]}
    p = tmp_path / "bad.ply"
    _write_foreign_ply(p, cols, "binary_little_endian", "float")
    with pytest.raises(ply.PlyError, match="missing"):
        ply.read_3dgs_ply(p)
    q = tmp_path / "notply.ply"
    q.write_bytes(b"solid stl\n")
    with pytest.raises(ply.PlyError):
        ply.read_3dgs_ply(q)


def test_render_only_conversion_matches_reference_test_values():
    """test/gaussians.jl:1-97: scales (1, 2, 3), a 90 degree rotation about z given as the
    unnormalised quaternion [sqrt(2)/2, 0, 0, sqrt(2)/2] -> covariance diag(4, 1, 9); identity
    quaternions [1, 0, 0, 0] -> diag(s^2); opacity logit 0.5 -> 0.622459331."""
    s2 = np.sqrt(2) / 2
    g = host.HostGaussians(
        np.array([[1, 2, 3, 0.5], [4, 5, 6, 0.25], [7, 8, 9, 0.75]], dtype=f32),
        np.log(np.array([[1, 2, 3], [4, 5, 6], [7, 8, 9]], dtype=f32)).astype(f32),
        np.array([[s2, 0, 0, s2], [1, 0, 0, 0], [1, 0, 0, 0]], dtype=f32),
        np.ones((3, 3, 1), dtype=f32))
    ro = ply.to_render_only(g)
    np.testing.assert_allclose(ro.means_opacity[:, 3], [0.622459331, 0.5621765, 0.6791787], rtol=1e-6)
    np.testing.assert_array_equal(ro.means_opacity[:, :3], g.means_opacity[:, :3])
    np.testing.assert_allclose(ro.covariances[0], [4, 0, 0, 1, 0, 9], atol=2e-6)
    np.testing.assert_allclose(ro.covariances[1], [16, 0, 0, 25, 0, 36], rtol=1e-6)
    np.testing.assert_allclose(ro.covariances[2], [49, 0, 0, 64, 0, 81], rtol=1e-6)
    R = ply.quaternion_to_rotation_matrix(g.rotation[:1])[0]
    np.testing.assert_allclose(R, [[0, -1, 0], [1, 0, 0], [0, 0, 1]], atol=1e-7)


def test_covariances_match_scipy_rotations():
    from scipy.spatial.transform import Rotation
    rng = np.random.default_rng(5)
    q = rng.standard_normal((500, 4)).astype(f32) * 3
    s = (rng.standard_normal((500, 3)) * 0.5).astype(f32)
    cov = ply.scaling_rotation_to_covariances(s, q)
    R = Rotation.from_quat(q[:, [1, 2, 3, 0]].astype(np.float64)).as_matrix()  # scalar-last
    V = np.einsum("nij,nj,nkj->nik", R, np.exp(2 * s.astype(np.float64)), R)
    ref = np.stack([V[:, 0, 0], V[:, 1, 0], V[:, 2, 0], V[:, 1, 1], V[:, 2, 1], V[:, 2, 2]], axis=1)
    scale = np.abs(V).max(axis=(1, 2))[:, None]
    assert np.max(np.abs(cov - ref) / scale) < 1e-5


def _camera_entry(**kw):
    e = {"id": 0, "img_name": "00000", "width": 1001, "height": 500,
         "position": [0.5, -1.25, 3.0], "rotation": [[0, 1, 0], [-1, 0, 0], [0, 0, 1]],
         "fy": 700.0, "fx": 710.0}
    e.update(kw)
    return e


def test_cameras_json_original_3dgs_entry(tmp_path):
    p = tmp_path / "cameras.json"
    p.write_text(json.dumps([_camera_entry()]))
    (c,) = ply.load_cameras_from_json(p)
    assert (c.width, c.height) == (1001, 500)
    assert (c.fx, c.fy, c.skew) == (f32(710), f32(700), 0)
    assert (c.ppx, c.ppy) == (f32(500.5), f32(250))
    assert c.near_z == f32(0.2) and np.isinf(c.far_z)
    np.testing.assert_array_equal(c.R_c2w, [[0, 1, 0], [-1, 0, 0], [0, 0, 1]])  # rows
    np.testing.assert_array_equal(c.t_c2w, f32([0.5, -1.25, 3.0]))


def test_cameras_json_rescale_and_ppy_quirk(tmp_path):
    p = tmp_path / "cameras.json"
    p.write_text(json.dumps([_camera_entry(ppx=480.0, ppy=260.0, skew=2.0, near_z=0.5, far_z=100.0)]))
    (c,) = ply.load_cameras_from_json(p, rescale_factor=0.5)
    assert (c.width, c.height) == (500, 250)  # round(500.5) is 500: ties to even
    sx, sy = f32(f32(500) / f32(1001)), f32(0.5)
    assert c.fx == f32(f32(710) * sx) and c.fy == f32(f32(700) * sy)
    assert c.skew == f32(f32(2) * sx) and c.ppx == f32(f32(480) * sx)
    assert c.ppy == f32(f32(260) * sx)  # scaled by the x factor, as cameras.jl:478
    assert c.near_z == f32(0.5) and c.far_z == f32(100)
    (d,) = ply.load_cameras_from_json(p, forced_width=320, forced_height=240)
    assert (d.width, d.height) == (320, 240)
    assert d.fy == f32(f32(700) * f32(f32(240) / f32(500)))


def test_cameras_json_round_trip(tmp_path):
    cams = [host.look_at_camera(640, 480, 60, (3.0, -1.0, -4.0)),
            host.look_at_camera(300, 200, 75, (-2.0, 0.5, 5.0), target=(0.1, 0.2, 0.3))]
    p = tmp_path / "cameras.json"
    ply.save_cameras_json(p, cams)
    entries = json.loads(p.read_text())
    assert list(entries[0]) == ["width", "height", "fx", "fy", "skew", "ppx", "ppy", "position", "rotation"]
    back = ply.load_cameras_from_json(p)
    for a, b in zip(cams, back):
        assert (a.width, a.height, a.fx, a.fy, a.skew, a.ppx, a.ppy) == (b.width, b.height, b.fx, b.fy, b.skew,
                                                                       b.ppx, b.ppy)
        np.testing.assert_array_equal(a.R_c2w, b.R_c2w)
        np.testing.assert_array_equal(a.t_c2w, b.t_c2w)
        np.testing.assert_array_equal(a.P, b.P)


def test_oracle_render_only_close_to_trainable(oracle, tmp_path):
    """The oracle's render-only projection (J V J^T from the file's covariances) against its
    trainable projection (J R S from the features), which the reference goldens pin: they
    differ only in float32 rounding, so integer outputs agree and images within 1e-4."""
    from tdgs_amd import synthetic
    w = synthetic.config(0, n=3000)
    p = tmp_path / "model.ply"
    ply.save_3dgs_ply(p, w.gaussians)
    cam = w.cameras[0]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, 0)
    a = oracle.render(ply.read_3dgs_ply(p), cam, t, opts)
    b = oracle.render(ply.read_render_only_ply(p), cam, t, opts)
    assert a["nb_fgaussians"] == b["nb_fgaussians"] > 1000
    assert abs(a["nb_keys"] - b["nb_keys"]) <= a["nb_keys"] // 1000
    d = np.abs(a["rgb"] - b["rgb"])
    assert d.mean() < 1e-6 and np.quantile(d, 0.999) < 1e-4
