"""MI355X-native render/train core for 3D Gaussian Splatting (host-side mirror).

The package directory name contains a dot, so it is loaded by path; see
__graft_entry__.load_package(), which registers it as the module ``tdgs_amd``.
"""
from . import abi, host  # noqa: F401
