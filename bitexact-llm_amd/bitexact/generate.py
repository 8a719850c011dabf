"""Logits hashes (src/bitexact/generate.py:21-23)."""

import hashlib


def logits_sha(row):
    """SHA-256 (hex) of one int64 logits row: equal hashes <=> bit-identical logits."""
    return hashlib.sha256(row.contiguous().cpu().numpy().tobytes()).hexdigest()
