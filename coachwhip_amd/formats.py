"""GGUF block formats on the expert path: type ids, weights per block, bytes per block.

Type ids are GGUF's (vendor/candle-core/src/quantized/mod.rs:314-339), plus 21 (IQ3_S) and
22 (IQ2_S), which the reference's Metal shaders implement (quantized.metal:232-257) but its
type enum does not. Sizes: k_quants.rs:125-200, 631-635, 2959-2968; quantized.metal:217-296.
"""
F32, F16 = 0, 1
Q8_0 = 8
Q2_K = 10
Q3_K = 11
Q4_K = 12
Q5_K = 13
Q6_K = 14
Q8_K = 15
IQ2_XXS = 16
IQ3_XXS = 18
IQ3_S = 21
IQ2_S = 22
IQ4_XS = 23
MXFP4 = 39
# not a GGUF type: MXFP4 blocks with each matrix's rows in groups of 16, the group's blocks of each
# 4-block step side by side (the library's CW_MXFP4_R16, made on the device by ExpertBank.rows16)
MXFP4_R16 = 295

NAMES = {F32: "f32", F16: "f16", Q8_0: "q8_0", Q2_K: "q2_K", Q3_K: "q3_K", Q4_K: "q4_K", Q5_K: "q5_K",
         Q6_K: "q6_K", Q8_K: "q8_K", IQ2_XXS: "iq2_xxs", IQ3_XXS: "iq3_xxs", IQ3_S: "iq3_s", IQ2_S: "iq2_s",
         IQ4_XS: "iq4_xs", MXFP4: "mxfp4", MXFP4_R16: "mxfp4_r16"}
BY_NAME = {v: k for k, v in NAMES.items()}

_BLOCK = {F32: 1, F16: 1, Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_K: 256,
          IQ2_XXS: 256, IQ3_XXS: 256, IQ3_S: 256, IQ2_S: 256, IQ4_XS: 256, MXFP4: 32, MXFP4_R16: 32}
_SIZE = {F32: 4, F16: 2, Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 292,
         IQ2_XXS: 66, IQ3_XXS: 98, IQ3_S: 110, IQ2_S: 82, IQ4_XS: 136, MXFP4: 17, MXFP4_R16: 17}
# byte offset of the f16 super-block (or block) scale d
D_OFFSET = {Q8_0: 0, Q2_K: 80, Q3_K: 108, Q4_K: 0, Q5_K: 0, Q6_K: 208, IQ2_XXS: 0, IQ3_XXS: 0, IQ3_S: 0,
            IQ2_S: 0, IQ4_XS: 0}

# the sources of the shrink to Q2_K (crates/engine/src/requant.rs:334-352)
SHRINK_SOURCES = (Q3_K, Q4_K, Q5_K)

# the weight formats the kernels take (Q8_K is an activation format only)
WEIGHT_TYPES = (Q8_0, Q2_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ2_S, IQ3_XXS, IQ3_S, IQ4_XS, MXFP4)


def block_size(dtype):
    return _BLOCK[dtype]


def type_size(dtype):
    return _SIZE[dtype]


def row_bytes(dtype, k):
    bs = _BLOCK[dtype]
    if k % bs:
        raise ValueError("%s rows need a multiple of %d weights, got %d" % (NAMES[dtype], bs, k))
    return k // bs * _SIZE[dtype]


def matrix_bytes(dtype, n, k):
    if dtype == MXFP4_R16:  # whole groups of 16 rows
        n = (n + 15) // 16 * 16
    return n * row_bytes(dtype, k)


def rows16_offset(r, b, nblk):
    """Byte offset of block b of row r in an MXFP4_R16 matrix of nblk blocks per row: group r // 16
    holds its 16 rows' bytes; within it step c (blocks 4c .. 4c + cb - 1) holds the 16 rows' blocks
    of that step side by side, row after row."""
    c = b // 4
    cb = min(4, nblk - 4 * c)
    return (r // 16) * 16 * nblk * 17 + c * 1088 + (r % 16) * 17 * cb + (b % 4) * 17
