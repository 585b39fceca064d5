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


class GGUFError(ValueError):
    """Malformed or unsupported tensor data (the reference's gguf.GGUFError)."""


def block_info(fmt):
    """fmt: name or GGML id -> (id, name, values per block, bytes per block)."""
    t = TYPE_ID[fmt] if isinstance(fmt, str) else int(fmt)
    if t not in GGML_TYPES:
        raise GGUFError(f"tensor type {fmt} is not served by this library")
    name, bv, bb = GGML_TYPES[t]
    return t, name, bv, bb
