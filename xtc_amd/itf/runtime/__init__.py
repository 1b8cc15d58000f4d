# SPDX-License-Identifier: BSD-3-Clause
from .accelerator import AcceleratorDevice
from .common import CommonRuntimeInterface

__all__ = ["AcceleratorDevice", "CommonRuntimeInterface"]
