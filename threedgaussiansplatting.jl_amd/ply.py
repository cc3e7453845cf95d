"""3DGS model and camera files: the .ply reader/writer (src/gaussians.jl:553-592, 839-968) and
cameras.json (src/cameras.jl:403-522), host side.

PLY: one `vertex` element. Properties are read by name, in any order and of any numeric type
(binary little/big endian or ASCII). Written files are binary little endian, with the property
order of gaussians.jl:902-913 (x y z [nx ny nz] f_dc_0..2 f_rest_* opacity scale_0..2 rot_0..3;
the order matters to the SIBR viewer). f_rest_k is coefficient 1 + k % (h - 1) of colour
channel k // (h - 1): all red coefficients, then green, then blue.

cameras.json: a list of cameras with width, height, fx, fy, position and rotation (the
camera-to-world rotation as a list of rows); skew, ppx, ppy, near_z and far_z are optional
(0, centred principal point, 0.2, inf). Other keys (id, img_name) are ignored.
"""
from __future__ import annotations

import json
import math
import re

import numpy as np

from .host import DEFAULT_FAR, DEFAULT_NEAR, HostGaussians, HostRenderOnlyGaussians, PinholeCamera

f32 = np.float32

_PLY_TYPES = {
    "char": "i1", "int8": "i1", "uchar": "u1", "uint8": "u1",
    "short": "i2", "int16": "i2", "ushort": "u2", "uint16": "u2",
    "int": "i4", "int32": "i4", "uint": "u4", "uint32": "u4",
    "float": "f4", "float32": "f4", "double": "f8", "float64": "f8",
}


class PlyError(ValueError):
    pass


def read_ply_vertices(path) -> dict[str, np.ndarray]:
    """The `vertex` element of a .ply file as {property name: 1-D array}."""
    with open(path, "rb") as fh:
        if fh.readline().strip() != b"ply":
            raise PlyError(f"{path}: not a PLY file")
        fmt = None
        elements = []   # (name, count, [(prop, dtype)])
        while True:
            line = fh.readline()
            if not line:
                raise PlyError(f"{path}: header without end_header")
            words = line.decode("ascii", "replace").split()
            if not words or words[0] in ("comment", "obj_info"):
                continue
            if words[0] == "format":
                fmt = words[1]
            elif words[0] == "element":
                elements.append((words[1], int(words[2]), []))
            elif words[0] == "property":
                if words[1] == "list":  # faces and the like; only a problem ahead of the vertices
                    elements[-1][2].append((words[-1], None))
                    continue
                if words[1] not in _PLY_TYPES:
                    raise PlyError(f"{path}: unknown property type {words[1]}")
                elements[-1][2].append((words[2], _PLY_TYPES[words[1]]))
            elif words[0] == "end_header":
                break
        if fmt not in ("binary_little_endian", "binary_big_endian", "ascii"):
            raise PlyError(f"{path}: unsupported format {fmt}")
        out = None
        for name, count, props in elements:
            if any(t is None for _, t in props):
                if fmt == "ascii" and name != "vertex":
                    for _ in range(count):
                        fh.readline()
                    continue
                raise PlyError(f"{path}: list property in element {name} ahead of the vertex data")
            if fmt == "ascii":
                rows = [fh.readline().split() for _ in range(count)]
                data = {p: np.array([float(r[i]) for r in rows], dtype=t) for i, (p, t) in enumerate(props)}
            else:
                order = "<" if fmt == "binary_little_endian" else ">"
                dt = np.dtype([(p, order + t) for p, t in props])
                raw = np.frombuffer(fh.read(dt.itemsize * count), dtype=dt, count=count)
                data = {p: raw[p].astype(raw[p].dtype.newbyteorder("=")) for p, _ in props}
            if name == "vertex":
                out = data
                break
        if out is None:
            raise PlyError(f"{path}: no vertex element")
        return out


def _f_rest_index(name):
    return int(name.rsplit("_", 1)[1])


def read_3dgs_ply(path) -> HostGaussians:
    """_read_3DGS_ply (gaussians.jl:553-592) into a HostGaussians (features: opacity logits,
    log-scales, unnormalised quaternions [r, x, y, z], SH coefficients (n, 3, h))."""
    v = read_ply_vertices(path)
    need = ["x", "y", "z", "opacity", "f_dc_0", "f_dc_1", "f_dc_2", "scale_0", "scale_1", "scale_2",
            "rot_0", "rot_1", "rot_2", "rot_3"]
    missing = [k for k in need if k not in v]
    if missing:
        raise PlyError(f"{path}: missing vertex properties {missing}")
    n = len(v["x"])
    rest = sorted((k for k in v if re.fullmatch(r"f_rest_\d+", k)), key=_f_rest_index)
    if len(rest) % 3:
        raise PlyError(f"{path}: {len(rest)} f_rest properties, not a multiple of 3")
    h = 1 + len(rest) // 3
    if int(round(math.sqrt(h))) ** 2 != h or h > 16:
        raise PlyError(f"{path}: {h} SH coefficients per channel is not (d+1)^2 for d <= 3")
    mo = np.stack([v["x"], v["y"], v["z"], v["opacity"]], axis=1).astype(f32)
    sc = np.stack([v["scale_0"], v["scale_1"], v["scale_2"]], axis=1).astype(f32)
    rot = np.stack([v["rot_0"], v["rot_1"], v["rot_2"], v["rot_3"]], axis=1).astype(f32)
    sh = np.empty((n, 3, h), dtype=f32)
    for c in range(3):
        sh[:, c, 0] = v[f"f_dc_{c}"]
        for i in range(1, h):
            sh[:, c, i] = v[rest[c * (h - 1) + i - 1]]
    return HostGaussians(np.ascontiguousarray(mo), np.ascontiguousarray(sc), np.ascontiguousarray(rot),
                         np.ascontiguousarray(sh))


def save_3dgs_ply(path, g: HostGaussians, force_sh_degree_3=False, include_normals=False, use_float_double=False):
    """save_to_ply (gaussians.jl:839-920): binary little endian, SIBR property order.
    force_sh_degree_3 pads the coefficients with zeros to degree 3; include_normals writes zero
    normals; use_float_double writes the type name `float` instead of `float32`."""
    n = g.n
    h = g.sh.shape[2]
    hw = 16 if force_sh_degree_3 else h
    cols = [("x", g.means_opacity[:, 0]), ("y", g.means_opacity[:, 1]), ("z", g.means_opacity[:, 2])]
    if include_normals:
        z = np.zeros(n, dtype=f32)
        cols += [("nx", z), ("ny", z), ("nz", z)]
    cols += [(f"f_dc_{c}", g.sh[:, c, 0]) for c in range(3)]
    for c in range(3):
        for i in range(1, hw):
            col = g.sh[:, c, i] if i < h else np.zeros(n, dtype=f32)
            cols.append((f"f_rest_{c * (hw - 1) + i - 1}", col))
    cols.append(("opacity", g.means_opacity[:, 3]))
    cols += [(f"scale_{i}", g.scaling[:, i]) for i in range(3)]
    cols += [(f"rot_{i}", g.rotation[:, i]) for i in range(4)]
    tname = "float" if use_float_double else "float32"
    header = ["ply", "format binary_little_endian 1.0", f"element vertex {n}"]
    header += [f"property {tname} {name}" for name, _ in cols]
    header.append("end_header")
    data = np.empty((n, len(cols)), dtype="<f4")
    for j, (_, col) in enumerate(cols):
        data[:, j] = col
    with open(path, "wb") as fh:
        fh.write(("\n".join(header) + "\n").encode("ascii"))
        fh.write(data.tobytes())


def quaternion_to_rotation_matrix(q):
    """misc.jl:133-141 in float32, for an (n, 4) array of [r, x, y, z] -> (n, 3, 3)."""
    q = np.asarray(q, dtype=f32)
    s = np.sqrt(f32(2) * (f32(1) / (q * q).sum(axis=1, dtype=f32))).astype(f32)
    r, x, y, z = (q * s[:, None]).astype(f32).T
    R = np.empty((q.shape[0], 3, 3), dtype=f32)
    R[:, 0, 0] = 1 - (y * y + z * z); R[:, 0, 1] = x * y - r * z; R[:, 0, 2] = x * z + r * y
    R[:, 1, 0] = x * y + r * z; R[:, 1, 1] = 1 - (x * x + z * z); R[:, 1, 2] = y * z - r * x
    R[:, 2, 0] = x * z - r * y; R[:, 2, 1] = y * z + r * x; R[:, 2, 2] = 1 - (x * x + y * y)
    return R


def scaling_rotation_to_covariances(scaling, rotation):
    """_scaling_rotation_features_to_covariances (gaussians.jl:467-483): lower halves
    [V11, V21, V31, V22, V32, V33] of (R S)(R S)^T, S = diag(exp(log-scales)), float32."""
    R = quaternion_to_rotation_matrix(rotation)
    RS = (R * np.exp(np.asarray(scaling, dtype=f32))[:, None, :]).astype(f32)
    V = np.einsum("nij,nkj->nik", RS, RS).astype(f32)
    return np.stack([V[:, 0, 0], V[:, 1, 0], V[:, 2, 0], V[:, 1, 1], V[:, 2, 1], V[:, 2, 2]], axis=1).astype(f32)


def to_render_only(g: HostGaussians) -> HostRenderOnlyGaussians:
    """RenderOnlyGaussiansVector(tgv) and RenderOnlyGaussiansVector(ply_path)
    (gaussians.jl:441-455, 741-762): means with sigmoid-activated opacities, covariances from
    the scaling and rotation features, the same SH coefficients."""
    mo = g.means_opacity.copy()
    mo[:, 3] = (f32(1) / (f32(1) + np.exp(-mo[:, 3]))).astype(f32)
    return HostRenderOnlyGaussians(mo, scaling_rotation_to_covariances(g.scaling, g.rotation), g.sh.copy())


def read_render_only_ply(path) -> HostRenderOnlyGaussians:
    """RenderOnlyGaussiansVector(ply_path) (gaussians.jl:741-762)."""
    return to_render_only(read_3dgs_ply(path))


def load_cameras_from_json(path, rescale_factor=None, forced_width=None, forced_height=None):
    """load_cameras_from_json (cameras.jl:403-505). With rescale_factor the size is rounded
    (ties to even, as Julia's round) and the intrinsics scaled; ppy is scaled by the x factor,
    as cameras.jl:470 does."""
    with open(path) as fh:
        entries = json.load(fh)
    cams = []
    for e in entries:
        if forced_width is not None:
            width = int(forced_width)
        else:
            width = int(e["width"]) if rescale_factor is None else int(round(e["width"] * rescale_factor))
        if forced_height is not None:
            height = int(forced_height)
        else:
            height = int(e["height"]) if rescale_factor is None else int(round(e["height"] * rescale_factor))
        sx = f32(f32(width) / f32(e["width"]))
        sy = f32(f32(height) / f32(e["height"]))
        fx = f32(f32(e["fx"]) * sx)
        fy = f32(f32(e["fy"]) * sy)
        skew = f32(f32(e["skew"]) * sx) if "skew" in e else f32(0)
        ppx = f32(f32(e["ppx"]) * sx) if "ppx" in e else f32(f32(width) / f32(2))
        ppy = f32(f32(e["ppy"]) * sx) if "ppy" in e else f32(f32(height) / f32(2))
        near = f32(e.get("near_z", DEFAULT_NEAR))
        far = f32(e.get("far_z", DEFAULT_FAR))
        R = np.asarray(e["rotation"], dtype=f32).reshape(3, 3)
        t = np.asarray(e["position"], dtype=f32).reshape(3)
        cams.append(PinholeCamera(width, height, fx, fy, skew, ppx, ppy, near, far, R, t))
    return cams


def save_cameras_json(path, cams):
    """save_json (cameras.jl:507-522): width, height, fx, fy, skew, ppx, ppy, position and the
    camera-to-world rotation as a list of rows."""
    out = []
    for c in cams:
        out.append({"width": int(c.width), "height": int(c.height), "fx": float(c.fx), "fy": float(c.fy),
                    "skew": float(c.skew), "ppx": float(c.ppx), "ppy": float(c.ppy),
                    "position": [float(v) for v in c.t_c2w],
                    "rotation": [[float(v) for v in row] for row in c.R_c2w]})
    with open(path, "w") as fh:
        json.dump(out, fh, indent=2)
