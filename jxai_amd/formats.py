"""GGML block formats used on the MoE expert path.

Type codes and block geometry follow the reference engine:
  - ``GGMLType`` enum values: include/common.h:45-77
  - block sizes / bytes per block: include/common.h:154-189
  - ``tensor_byte_size`` (rows hold ceil(cols/blk) whole blocks): include/common.h:191-195
  - packed block structs ``block_q4_0`` / ``block_q8_0`` / ``block_q4_K``: include/quant.h:10-33,
    ``block_q5_K`` / ``block_q6_K`` 36-50, ``block_q5_0`` 60-66
"""
from __future__ import annotations

F32 = 0
F16 = 1
Q4_0 = 2
Q5_0 = 6
Q8_0 = 8
Q4_K = 12
Q5_K = 13
Q6_K = 14
BF16 = 30

NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K",
         Q6_K: "Q6_K", BF16: "BF16"}
BY_NAME = {v: k for k, v in NAMES.items()}

# elements per block, bytes per block (include/common.h:154-189)
BLOCK = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144),
         Q5_K: (256, 176), Q6_K: (256, 210), BF16: (1, 2)}

EXPERT_TYPES = (Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K)
ROUTER_TYPES = (F32, F16, BF16)  # the router GEMV goes through matmul_quant_f32 (transformer.cpp:2591)
K_QUANTS = (Q4_K, Q5_K, Q6_K)


def blck_size(t: int) -> int:
    return BLOCK[t][0]


def type_size(t: int) -> int:
    return BLOCK[t][1]


def row_bytes(t: int, cols: int) -> int:
    """Bytes of one row of ``cols`` elements; partial blocks round up (common.h:191-195)."""
    b, s = BLOCK[t]
    return ((cols + b - 1) // b) * s


def matrix_bytes(t: int, rows: int, cols: int) -> int:
    return rows * row_bytes(t, cols)


def supports_q8_activation(t: int, cols: int) -> bool:
    """Whether the reference quantizes this matrix's input to Q8_0 (quant.cpp:3881-3893)."""
    if t in (Q4_0, Q8_0):
        return cols % 32 == 0
    if t in K_QUANTS:
        return cols % 256 == 0
    return False
