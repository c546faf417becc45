"""Golden-fixture cases: small shapes covering the reference tests' mask
families (test_mapped_attention.py), the BASELINE cfg1 shape, padding, GQA and
fully masked rows.  Masks are referenced by name so the fixtures stay data."""
import numpy as np

MASKS = {
    "causal": None,  # is_causal=True
    "sliding": lambda b, h, q, k: (q - 3 <= k) & (k <= q + 2),             # test_mapped_attention.py:1552
    "alternating": lambda h, q, k: ((q + k) % 2 == 0) | (q == k),
    "head_specific": lambda h, q, k: (q + 5 * h) >= k,
    "batch_doc": lambda b, h, q, k: (q // (7 + 3 * b)) == (k // (7 + 3 * b)),
    "local3": lambda h, q, k: abs(q - k) <= 2,                              # :1076-1112
    "late_rows": lambda b, h, q, k: (q > 20) & (k <= q),                    # rows 0..20 empty
}

CASES = {
    # BASELINE cfg1: causal fp32, B=2 L=128 H=8 d=64, block 32, N(0,1) inputs, forward only
    "cfg1_causal_fp32": dict(shape=(2, 128, 128, 8, 8, 64), mask="causal", block_size=32,
                             dtype="float32", seed=101, scaled=False, forward_only=True),
    "causal_bf16_gqa": dict(shape=(1, 96, 96, 4, 2, 64), mask="causal", block_size=32,
                            dtype="bfloat16", seed=102),
    "sliding_window_bf16": dict(shape=(1, 80, 80, 2, 2, 128), mask="sliding", block_size=16,
                                window_size=(3, 2), dtype="bfloat16", seed=103),
    "alternating_fp16": dict(shape=(1, 64, 64, 2, 2, 64), mask="alternating", block_size=16,
                             dtype="float16", seed=104),
    "head_specific_bf16": dict(shape=(1, 64, 64, 4, 4, 64), mask="head_specific", block_size=32,
                               dtype="bfloat16", seed=105),
    "batch_doc_bf16": dict(shape=(3, 50, 50, 2, 2, 64), mask="batch_doc", block_size=25,
                           dtype="bfloat16", seed=106),
    "padding_fp32": dict(shape=(1, 10, 13, 4, 4, 64), mask="local3", block_size=4,
                         dtype="float32", seed=107, scaled=False),
    "empty_rows_bf16": dict(shape=(1, 64, 64, 2, 2, 128), mask="late_rows", block_size=64,
                            dtype="bfloat16", seed=108),
}


def kwargs_of(c):
    kw = {}
    if c["mask"] == "causal":
        kw["is_causal"] = True
    else:
        kw["mask_fn"] = MASKS[c["mask"]]
    if c.get("block_size") is not None:
        kw["block_size"] = c["block_size"]
    if c.get("window_size") is not None:
        kw["window_size"] = tuple(c["window_size"])
    return kw


def encode(x, dtype):
    """Storage form of a dtype-representable float32 array: float32 itself, or
    the 16-bit patterns of bfloat16 (upper half of the float32 bits) / float16."""
    x = np.ascontiguousarray(x, np.float32)
    if dtype == "float32":
        return x
    if dtype == "float16":
        return x.astype(np.float16).view(np.uint16)
    assert dtype == "bfloat16"
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def decode(a, dtype):
    """Inverse of encode: float32 values."""
    if dtype == "float32":
        return np.asarray(a, np.float32)
    if dtype == "float16":
        return a.view(np.float16).astype(np.float32)
    return (a.astype(np.uint32) << 16).view(np.float32)


def round_to(x, dtype):
    """float32 array holding x rounded to dtype (round-to-nearest-even)."""
    import torch

    t = torch.from_numpy(np.asarray(x, np.float32))
    return t.to(getattr(torch, dtype)).float().numpy()
