"""rotatek_amd: MI355X-native (gfx950) RotateK decode hot path.

Drop-in for the reference package ``rotatek`` (beomseokg/rotatek,
rotatek/__init__.py:10-13):

    rotation.power_iteration_gpu   top-k eigenbasis of the Key covariance
    kernels.rotatek_decode         decode over rotated-truncated visual Keys
    kernels.full_channel_decode    full-width split-K decode (baseline)

The decode entry points follow ``ROTATEK_KERNEL`` (``paper`` | ``gqa``).
All GPU work runs in hand-written HIP kernels in ``librotatek_hip.so``
(build with ``python -m rotatek_amd.build``); ``install_as_rotatek()``
registers this package under the reference's module names so unmodified
callers (``from rotatek.kernels import rotatek_decode``) pick it up.
"""
import sys

from rotatek_amd.kernels import full_channel_decode, rotatek_decode
from rotatek_amd.rotation import power_iteration_gpu

__all__ = ["full_channel_decode", "rotatek_decode", "power_iteration_gpu", "install_as_rotatek"]


def install_as_rotatek() -> None:
    """Alias this package as ``rotatek`` / ``rotatek.kernels`` /
    ``rotatek.rotation`` / ``rotatek.baselines`` (and their submodules) in
    ``sys.modules``."""
    import rotatek_amd
    import rotatek_amd.kernels as k
    import rotatek_amd.kernels.fused_decode as fd
    import rotatek_amd.kernels.full_channel_flash_decoding as fc
    import rotatek_amd.kernels.gqa_decode as gd
    import rotatek_amd.baselines as bl
    import rotatek_amd.baselines.spark as bs
    import rotatek_amd.baselines.think as bt
    import rotatek_amd.rotation as rot
    sys.modules["rotatek"] = rotatek_amd
    sys.modules["rotatek.baselines"] = bl
    sys.modules["rotatek.baselines.think"] = bt
    sys.modules["rotatek.baselines.spark"] = bs
    sys.modules["rotatek.kernels"] = k
    sys.modules["rotatek.kernels.fused_decode"] = fd
    sys.modules["rotatek.kernels.full_channel_flash_decoding"] = fc
    sys.modules["rotatek.kernels.gqa_decode"] = gd
    sys.modules["rotatek.rotation"] = rot
