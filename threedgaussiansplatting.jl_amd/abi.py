"""ctypes mirrors of the plain-C structs declared in include/tdgs.h.

Field order and types follow the header exactly; both the product library (libtdgs.so) and
the CPU oracle take these structs by pointer.
"""
import ctypes as C

TDGS_OK = 0
TDGS_ERR_INVALID = 1
TDGS_ERR_CAPACITY = 2
TDGS_ERR_HIP = 3
TDGS_ERR_UNSUPPORTED = 4
TDGS_ERR_DEVICE = 5

TDGS_TRAINABLE = 0
TDGS_RENDER_ONLY = 1
TDGS_CLIP_CLAMP = 0
TDGS_CLIP_FILTER = 1
TDGS_FLAG_EXACT_SH_JACOBIAN = 0x1
TDGS_FLAG_EXACT_AA_GRADIENT = 0x2
TDGS_FLAG_DEVICE_COUNTS = 0x4
TDGS_FRAME_OK = 0
TDGS_FRAME_KEY_CAPACITY = 1
TDGS_FRAME_KEY_RANGE = 2
TDGS_IMAGE_RGB = 0
TDGS_IMAGE_TRANSMITTANCE = 1
TDGS_IMAGE_DEPTH = 2

fp = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int32)
i64p = C.POINTER(C.c_int64)
u8p = C.POINTER(C.c_uint8)


class Camera(C.Structure):
    _fields_ = [("width", C.c_int32), ("height", C.c_int32), ("P", C.c_float * 12),
                ("near_z", C.c_float), ("far_z", C.c_float), ("position", C.c_float * 3)]


class RenderOptionsC(C.Structure):
    _fields_ = [("background", C.c_float * 3), ("aa_min_factor", C.c_float),
                ("min_alpha", C.c_float), ("max_alpha", C.c_float),
                ("min_transmittance", C.c_float), ("dilation_x", C.c_float),
                ("dilation_y", C.c_float), ("clip_x_min", C.c_float), ("clip_x_max", C.c_float),
                ("clip_y_min", C.c_float), ("clip_y_max", C.c_float), ("sh_degree", C.c_int32),
                ("clip_mode", C.c_int32), ("antialiasing", C.c_int32), ("flags", C.c_int32)]


class TilingC(C.Structure):
    _fields_ = [("tile_width", C.c_int32), ("tile_height", C.c_int32),
                ("nb_tiles_x", C.c_int32), ("nb_tiles_y", C.c_int32)]


class Gaussians(C.Structure):
    _fields_ = [("kind", C.c_int32), ("n", C.c_int32), ("sh_degree", C.c_int32),
                ("reserved", C.c_int32), ("means_opacity", C.c_void_p), ("scaling", C.c_void_p),
                ("rotation", C.c_void_p), ("covariances", C.c_void_p), ("sh", C.c_void_p)]


class RenderBuffersC(C.Structure):
    _fields_ = [("capacity", C.c_int32), ("reserved", C.c_int32), ("key_capacity", C.c_int64),
                ("keep", C.c_void_p), ("fgidx_to_gidx", C.c_void_p), ("depths", C.c_void_p),
                ("f2d", C.c_void_p), ("tile_ranges", C.c_void_p), ("counts", C.c_void_p),
                ("keys", C.c_void_p), ("values", C.c_void_p), ("sorted_keys", C.c_void_p),
                ("sorted_values", C.c_void_p), ("tiles_end", C.c_void_p), ("temp", C.c_void_p),
                ("temp_bytes", C.c_size_t)]


class RenderOutputsC(C.Structure):
    _fields_ = [("rgb", C.c_void_p), ("T", C.c_void_p), ("depth", C.c_void_p), ("last", C.c_void_p)]


class GradientsC(C.Structure):
    _fields_ = [("capacity", C.c_int32), ("sh_degree", C.c_int32), ("grads2d", C.c_void_p),
                ("mean2d_grads", C.c_void_p), ("opacity_grads", C.c_void_p), ("licov2d_grads", C.c_void_p),
                ("color_grads", C.c_void_p), ("mean3d", C.c_void_p), ("opacity_feature", C.c_void_p),
                ("scaling_features", C.c_void_p), ("rotation_features", C.c_void_p),
                ("sh", C.c_void_p)]


class AdamStateC(C.Structure):
    _fields_ = [("means_moments", C.c_void_p), ("opacity_moments", C.c_void_p),
                ("scaling_moments", C.c_void_p), ("rotation_moments", C.c_void_p),
                ("sh_moments", C.c_void_p), ("lr_means", C.c_float), ("lr_opacity", C.c_float),
                ("lr_scaling", C.c_float), ("lr_rotation", C.c_float), ("lr_sh_dc", C.c_float),
                ("lr_sh_rest", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float),
                ("epsilon", C.c_float), ("update_count", C.c_int32)]


class AdcBuffersC(C.Structure):
    _fields_ = [("capacity", C.c_int32), ("new_capacity", C.c_int32),
                ("accum_grad_norms", C.c_void_p), ("contribution_counts", C.c_void_p),
                ("prune", C.c_void_p), ("densify", C.c_void_p), ("clone", C.c_void_p),
                ("new_counts_cs", C.c_void_p), ("ngidx_to_gidx", C.c_void_p),
                ("temp", C.c_void_p), ("temp_bytes", C.c_size_t)]


def sh_coeffs_per_channel(degree: int) -> int:
    return (int(degree) + 1) ** 2
