"""Viewer output (convert_*_to_gl_img_kernel!, gui.jl:958-1067) through the C-ABI: known
values pin the rounding (to nearest, ties to even), the clamps, the orientation of the depth
ramp, and the transposition from column-major h x w to row-major 3 x w x h bytes."""
import numpy as np
import pytest
import torch

from tdgs_amd import abi

pytestmark = pytest.mark.gpu

f32 = np.float32


def _u8(gpu, img, kind, dmin=0.0, dmax=1.0):
    t = torch.from_numpy(np.ascontiguousarray(img)).cuda()
    out = gpu.image_to_rgb8(t, kind, dmin, dmax)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_rgb_known_values(gpu):
    vals = f32([0.0, 1.0, 2.0, 0.5, 1.5 / 255, 2.5 / 255, 254.5 / 255, 1e-3, 0.999])
    want = [0, 255, 255, 128, 2, 2, 254, 0, 255]   # 127.5 -> 128, 1.5 -> 2, 2.5 -> 2 (even)
    img = np.zeros((len(vals), 1, 3), f32)         # w = len(vals), h = 1
    img[:, 0, 0] = vals
    img[:, 0, 1] = vals[::-1]
    out = _u8(gpu, img, abi.TDGS_IMAGE_RGB)
    assert out.shape == (1, len(vals), 3)
    assert out[0, :, 0].tolist() == [int(np.round(f32(v) * f32(255))) if v <= 1 else 255 for v in vals]
    assert out[0, :, 0].tolist() == want
    assert out[0, :, 1].tolist() == want[::-1]
    assert out[0, :, 2].tolist() == [0] * len(vals)


def test_transmittance_and_depth_known_values(gpu):
    T = f32([[0.0, 0.25], [1.0, 0.5]])             # (w=2, h=2)
    out = _u8(gpu, T, abi.TDGS_IMAGE_TRANSMITTANCE)
    # out[y, x, c] = T[x, y]
    assert out[:, :, 0].tolist() == [[0, 255], [64, 128]]
    assert (out[:, :, 0] == out[:, :, 2]).all()
    d = f32([[1.0, 3.0, np.inf, 0.5, 2.0]]).T      # (w=5, h=1), range [1, 3]
    out = _u8(gpu, d.reshape(5, 1), abi.TDGS_IMAGE_DEPTH, 1.0, 3.0)
    assert out[0, :, 1].tolist() == [255, 0, 0, 255, 128]   # near white, far black; 127.5 -> 128


def test_transposition_large_ragged(gpu):
    w, h = 1000, 333
    rng = np.random.default_rng(3)
    img = rng.random((w, h, 3), dtype=np.float32) * f32(1.2)
    out = _u8(gpu, img, abi.TDGS_IMAGE_RGB)
    ref = np.where(img <= 1, np.rint(img * f32(255)), 255).astype(np.uint8).transpose(1, 0, 2)
    np.testing.assert_array_equal(out, ref)


def test_bad_arguments(gpu):
    t = torch.zeros((4, 4), device="cuda")
    with pytest.raises(gpu.TdgsError, match="min_depth"):
        gpu.image_to_rgb8(t, abi.TDGS_IMAGE_DEPTH, 2.0, 1.0)
    with pytest.raises(ValueError):
        gpu.image_to_rgb8(t, abi.TDGS_IMAGE_RGB)
