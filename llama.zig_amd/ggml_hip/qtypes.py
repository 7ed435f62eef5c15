"""ggml type ids and block geometry for the types on this path.

Ids as ggml numbers them (recorded in the reference's goldens,
src/ggml/quants/golden.zig:74-133); block sizes from
src/ggml/quants/blocks.zig:67-222.
"""
TYPE_F32 = 0
TYPE_Q4_0 = 2
TYPE_IQ4_XS = 23
TYPE_Q8_0 = 8
TYPE_Q8_1 = 9
TYPE_Q4_K = 12
TYPE_Q5_K = 13
TYPE_Q6_K = 14
TYPE_Q8_K = 15

TYPE_IDS = {"F32": TYPE_F32, "Q4_0": TYPE_Q4_0, "IQ4_XS": TYPE_IQ4_XS, "Q8_0": TYPE_Q8_0, "Q8_1": TYPE_Q8_1, "Q4_K": TYPE_Q4_K, "Q5_K": TYPE_Q5_K,
            "Q6_K": TYPE_Q6_K, "Q8_K": TYPE_Q8_K}
TYPE_NAMES = {v: k for k, v in TYPE_IDS.items()}

# elements per block, bytes per block
BLOCK = {TYPE_F32: (1, 4), TYPE_Q4_0: (32, 18), TYPE_IQ4_XS: (256, 136), TYPE_Q8_0: (32, 34), TYPE_Q8_1: (32, 36), TYPE_Q4_K: (256, 144), TYPE_Q5_K: (256, 176),
         TYPE_Q6_K: (256, 210), TYPE_Q8_K: (256, 292)}


def row_size(t: int, ne: int) -> int:
    """ggml_row_size: bytes of `ne` elements of type t (ne a multiple of the block)."""
    bs, ts = BLOCK[t]
    if ne % bs:
        raise ValueError(f"{ne} elements is not a whole number of {TYPE_NAMES[t]} blocks")
    return ne // bs * ts
