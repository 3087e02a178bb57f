"""The sibling estimate of the reference's M30 (seedpack/siblings.py:51-77, _Est): for a tensor seen
in several versions (quantizations of one model), the precision-weighted mean of the versions so far,
x = sum(x_i / h_i^2) / sum(1 / h_i^2) with h = sum(1 / h_i^2)^-1/2, h_i half the interval a version's
code stands for; it is the explicit (x, h) seed the next version is QR-coded against."""
import numpy as np

from . import device as dev
from ._lib import check, lib


def half_step(x, lo, hi, stream=None):
    """half the interval of each weight's code from its bounds (one infinite side: the finite one;
    none: -1, no information) -> float32 DeviceArray"""
    h = dev.DeviceArray(x.size, np.float32)
    check(lib().spa_est_half_step(x.ptr, lo.ptr, hi.ptr, x.size, h.ptr, stream))
    return h


class Est:
    """running sums of one slice's versions (device float32)"""

    def __init__(self, nw, stream=None):
        self.nw, self.stream = nw, stream
        self.ws = dev.DeviceArray(nw, np.float32).zero(stream)
        self.wx = dev.DeviceArray(nw, np.float32).zero(stream)
        self.x0 = None

    def add(self, x, h):
        """a version's values x and half steps h (float32 DeviceArrays of nw)"""
        if self.x0 is None:
            self.x0 = x
        check(lib().spa_est_add(x.ptr, h.ptr, self.nw, self.ws.ptr, self.wx.ptr, self.stream))

    def seed(self):
        """the explicit seed: float32 (x, h) per weight -> DeviceArray of 2 nw"""
        out = dev.DeviceArray(2 * self.nw, np.float32)
        x0 = self.x0 if self.x0 is not None else dev.DeviceArray(self.nw, np.float32).zero(self.stream)
        check(lib().spa_est_seed(self.ws.ptr, self.wx.ptr, x0.ptr, self.nw, out.ptr, self.stream))
        return out
