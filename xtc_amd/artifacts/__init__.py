# SPDX-License-Identifier: BSD-3-Clause
"""Named operation sizes for `loop-explore --op-name NAME`
(src/xtc/artifacts/operations.py:20-71, populated by
register_ttile_operations.py and register_subgraph_operations.py).

A name selects one operator instance by the layer it comes from
("ResNet18_04", "Gemma9B_FC", ...).  Each entry holds `dims` (the operator's
loop sizes in its dimension order) and `params` (conv strides).  Names match
case-insensitively; listing order is registration order, as in the
reference: the conv layers of Yolo9000, MobileNet and ResNet18, the matmuls
of transformer and Polybench shapes (src/xtc/schedules/ttile/prob_sizes.py),
then the SqueezeNet and AlexNet layers (src/xtc/artifacts/subgraph_sizes.py).
The sizes are the reference's; the table format is this module's own.
"""

from __future__ import annotations

import logging

__all__ = ["register_operation", "get_operation", "has_operation", "list_operations"]

logger = logging.getLogger(__name__)

_REGISTRY: dict[str, dict[str, dict]] = {}

CONV_DIMS = ("n", "h", "w", "f", "r", "s", "c")
MATMUL_DIMS = ("i", "j", "k")


def register_operation(operator: str, name: str, dims: dict[str, int], params: dict[str, int] | None = None) -> None:
    ops = _REGISTRY.setdefault(operator, {})
    key = name.lower()
    if key in ops:
        logger.warning("operation %s/%s is already registered", operator, key)
    ops[key] = {"name": name, "dims": dict(dims), "params": dict(params or {})}


def get_operation(operator: str, name: str) -> dict:
    if operator not in _REGISTRY:
        raise ValueError(f"operator {operator} not registered in operation registry")
    op = _REGISTRY[operator].get(name.lower())
    if op is None:
        raise ValueError(f"operation name {name} for operator {operator} not registered in operation registry")
    return op


def has_operation(operator: str, name: str) -> bool:
    return operator in _REGISTRY and name.lower() in _REGISTRY[operator]


def list_operations(operator: str = "") -> list[tuple[str, str]]:
    if not operator:
        return [(o, op["name"]) for o in _REGISTRY for op in _REGISTRY[o].values()]
    if operator not in _REGISTRY:
        raise ValueError(f"operator {operator} not registered in operation registry")
    return [(operator, op["name"]) for op in _REGISTRY[operator].values()]


# conv2d: name -> (n, h, w, f, r, s, c, SH, SW); h, w are output sizes
_CONV_TTILE = {
    "Yolo9000_00": (1, 544, 544, 32, 3, 3, 3, 1, 1),
    "Yolo9000_02": (1, 272, 272, 64, 3, 3, 32, 1, 1),
    "Yolo9000_04": (1, 136, 136, 128, 3, 3, 64, 1, 1),
    "Yolo9000_05": (1, 136, 136, 64, 1, 1, 128, 1, 1),
    "Yolo9000_08": (1, 68, 68, 256, 3, 3, 128, 1, 1),
    "Yolo9000_09": (1, 68, 68, 128, 1, 1, 256, 1, 1),
    "Yolo9000_12": (1, 34, 34, 512, 3, 3, 256, 1, 1),
    "Yolo9000_13": (1, 34, 34, 256, 1, 1, 512, 1, 1),
    "Yolo9000_18": (1, 17, 17, 1024, 3, 3, 512, 1, 1),
    "Yolo9000_19": (1, 17, 17, 512, 1, 1, 1024, 1, 1),
    "Yolo9000_23": (1, 17, 17, 28272, 1, 1, 1024, 1, 1),
    "MobilNet_01": (1, 112, 112, 32, 3, 3, 32, 1, 1),
    "MobilNet_02": (1, 112, 112, 64, 3, 3, 64, 2, 2),
    "MobilNet_03": (1, 56, 56, 128, 3, 3, 128, 1, 1),
    "MobilNet_04": (1, 56, 56, 128, 3, 3, 128, 2, 2),
    "MobilNet_05": (1, 28, 28, 256, 3, 3, 256, 1, 1),
    "MobilNet_06": (1, 28, 28, 256, 3, 3, 256, 2, 2),
    "MobilNet_07": (1, 14, 14, 512, 3, 3, 512, 1, 1),
    "MobilNet_08": (1, 14, 14, 512, 3, 3, 512, 2, 2),
    "MobilNet_09": (1, 7, 7, 1024, 3, 3, 1024, 1, 1),
    "ResNet18_01": (1, 224, 224, 64, 7, 7, 3, 2, 2),
    "ResNet18_02": (1, 56, 56, 64, 3, 3, 64, 1, 1),
    "ResNet18_03": (1, 56, 56, 64, 1, 1, 64, 1, 1),
    "ResNet18_04": (1, 56, 56, 128, 3, 3, 64, 2, 2),
    "ResNet18_05": (1, 56, 56, 128, 1, 1, 64, 2, 2),
    "ResNet18_06": (1, 28, 28, 128, 3, 3, 128, 1, 1),
    "ResNet18_07": (1, 28, 28, 256, 3, 3, 128, 2, 2),
    "ResNet18_08": (1, 28, 28, 256, 3, 3, 128, 1, 1),
    "ResNet18_09": (1, 14, 14, 256, 3, 3, 256, 1, 1),
    "ResNet18_10": (1, 14, 14, 512, 3, 3, 512, 2, 2),
    "ResNet18_11": (1, 14, 14, 512, 1, 1, 256, 2, 2),
    "ResNet18_12": (1, 7, 7, 512, 3, 3, 512, 1, 1),
}

# matmul: name -> (i, j, k)
_MATMUL_TTILE = {
    "Llama3AttMm": (8192, 8192, 4096),
    "Polybench_medium": (200, 224, 240),
    "Polybench_large": (1000, 1104, 1200),
    "Polybench_extralarge": (2000, 2304, 2600),
    "Llama3_In": (4096, 4096, 128),
    "Llama3_QK": (128, 4096, 8192),
    "Llama3_QKV": (128, 8192, 4096),
    "Llama3_FC": (4096, 4096, 4096),
    "Gemma27B_In": (4608, 4096, 256),
    "Gemma27B_QK": (256, 4608, 8192),
    "Gemma27B_QKV": (256, 8192, 4608),
    "Gemma27B_FC": (4608, 36864, 4608),
    "Gemma9B_In": (3584, 4096, 256),
    "Gemma9B_QK": (256, 3584, 8192),
    "Gemma9B_QKV": (256, 8192, 3584),
    "Gemma9B_FC": (3584, 14336, 3584),
    "Gemma7B_In": (3072, 4096, 256),
    "Gemma7B_QK": (256, 3072, 8192),
    "Gemma7B_QKV": (256, 8192, 3072),
    "Gemma7B_FC": (3072, 24576, 3072),
    "Gemma2B_In": (2048, 4096, 256),
    "Gemma2B_QK": (256, 2048, 8192),
    "Gemma2B_QKV": (256, 8192, 2048),
    "Gemma2B_FC": (2048, 16384, 2048),
}

_CONV_SUBGRAPH = {
    "SqueezeNet_00": (1, 224, 224, 96, 7, 7, 3, 2, 2),
    "SqueezeNet_01": (1, 54, 54, 16, 1, 1, 96, 1, 1),
    "SqueezeNet_03": (1, 56, 56, 64, 3, 3, 16, 1, 1),
    "SqueezeNet_04": (1, 54, 54, 16, 1, 1, 128, 1, 1),
    "SqueezeNet_05": (1, 54, 54, 32, 1, 1, 128, 1, 1),
    "SqueezeNet_07": (1, 54, 54, 128, 3, 3, 32, 1, 1),
    "SqueezeNet_08": (1, 27, 27, 32, 1, 1, 256, 1, 1),
    "SqueezeNet_11": (1, 27, 27, 48, 1, 1, 256, 1, 1),
    "SqueezeNet_13": (1, 27, 27, 192, 3, 3, 48, 1, 1),
    "SqueezeNet_14": (1, 27, 27, 48, 1, 1, 384, 1, 1),
    "SqueezeNet_17": (1, 27, 27, 256, 3, 3, 64, 1, 1),
    "SqueezeNet_21": (1, 15, 15, 1000, 1, 1, 512, 1, 1),
    "AlexNet_00": (1, 228, 228, 64, 11, 11, 3, 4, 4),
    "AlexNet_01": (1, 31, 31, 192, 5, 5, 64, 1, 1),
    "AlexNet_02": (1, 15, 15, 384, 3, 3, 192, 1, 1),
    "AlexNet_03": (1, 15, 15, 256, 3, 3, 384, 1, 1),
    "AlexNet_04": (1, 15, 15, 256, 3, 3, 256, 1, 1),
}

_MATMUL_SUBGRAPH = {
    "AlexNet_FC6": (1, 4096, 9216),
    "AlexNet_FC7": (1, 4096, 4096),
    "AlexNet_FC8": (1, 1000, 4096),
}


def _register(convs: dict[str, tuple[int, ...]], matmuls: dict[str, tuple[int, ...]]) -> None:
    for name, v in convs.items():
        register_operation("conv2d", name, dict(zip(CONV_DIMS, v[:7])), {"SH": v[7], "SW": v[8]})
    for name, v in matmuls.items():
        register_operation("matmul", name, dict(zip(MATMUL_DIMS, v)))


_register(_CONV_TTILE, _MATMUL_TTILE)
_register(_CONV_SUBGRAPH, _MATMUL_SUBGRAPH)
