"""GGUF block formats of the hot path: type ids, block geometry (GgmlType, src/quant/mod.rs:11-54)."""

Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ3_S, IQ4_XS = 8, 10, 11, 12, 13, 14, 16, 21, 23

NAMES = {Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K",
         IQ2_XXS: "IQ2_XXS", IQ3_S: "IQ3_S", IQ4_XS: "IQ4_XS"}
BY_NAME = {v: k for k, v in NAMES.items()}
# block_bytes, src/quant/mod.rs:40-43
BLOCK_BYTES = {Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ2_XXS: 66, IQ3_S: 110, IQ4_XS: 136}
# Offsets of the f16 super-block scales (d, and dmin where the format has one), as the reference's
# int_dots_match_dequant test sets them (src/cpu_moe.rs:1610).
F16_FIELDS = {Q8_0: (0,), Q2_K: (80, 82), Q3_K: (108,), Q4_K: (0, 2), Q5_K: (0, 2), Q6_K: (208,),
              IQ2_XXS: (0,), IQ3_S: (0,), IQ4_XS: (0,)}
TYPES = tuple(NAMES)


def block_elems(ty):
    return 32 if ty == Q8_0 else 256


def block_bytes(ty):
    return BLOCK_BYTES[ty]


def row_bytes(ty, cols):
    """GgmlType::row_bytes, src/quant/mod.rs:47."""
    return cols // block_elems(ty) * BLOCK_BYTES[ty]


def name(ty):
    return NAMES[ty]
