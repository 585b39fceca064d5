"""GGML tensor types of the formats this library serves: id -> (name, values per block, bytes per
block).  Same ids and sizes as the reference table ggufengine/gguf.py:64-78 (GGML_TYPES), which
follows ggml; the other formats of that table are outside this path."""

GGML_TYPES = {
    2: ("Q4_0", 32, 18),
    8: ("Q8_0", 32, 34),
    12: ("Q4_K", 256, 144),
    14: ("Q6_K", 256, 210),
    16: ("IQ2_XXS", 256, 66),
    35: ("TQ2_0", 256, 66),
}
TYPE_ID = {name: t for t, (name, _, _) in GGML_TYPES.items()}

# Every tensor type a GGUF file may hold (ggml's type traits: values and bytes per block), so that the
# reader can size and place tensors of all formats, including the float ones that stay on the CPU
# path (norms, embeddings).  Ids 142, 143 are a fork's 128-value variants of Q2_0 / TQ1_0.
GGML_ALL_TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22),
    7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36), 10: ("Q2_K", 256, 84),
    11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210),
    15: ("Q8_K", 256, 292), 16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98),
    19: ("IQ1_S", 256, 50), 20: ("IQ4_NL", 32, 18), 21: ("IQ3_S", 256, 110), 22: ("IQ2_S", 256, 82),
    23: ("IQ4_XS", 256, 136), 24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4), 27: ("I64", 1, 8),
    28: ("F64", 1, 8), 29: ("IQ1_M", 256, 56), 30: ("BF16", 1, 2), 34: ("TQ1_0", 256, 54),
    35: ("TQ2_0", 256, 66), 39: ("MXFP4", 32, 17), 41: ("Q1_0", 128, 18), 42: ("Q2_0", 64, 18),
    142: ("PQ2_0", 128, 34), 143: ("PTQ1_0", 128, 28),
}


class GGUFError(ValueError):
    """Malformed or unsupported tensor data (the reference's gguf.GGUFError)."""


def block_info(fmt):
    """fmt: name or GGML id -> (id, name, values per block, bytes per block)."""
    t = TYPE_ID[fmt] if isinstance(fmt, str) else int(fmt)
    if t not in GGML_TYPES:
        raise GGUFError(f"tensor type {fmt} is not served by this library")
    name, bv, bb = GGML_TYPES[t]
    return t, name, bv, bb
