"""Restatement of the offline weight repack (numpy).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

No reference counterpart: the reference consumes int4 weights packed as
byte j of each column = element 2j (low nibble) | element 2j+1 (high
nibble) (docs/Task1.md:78-81). The MFMA order defined by this build stores,
for every run of 8 consecutive elements of a column, byte i = (u[i] ^ 8) |
(u[i+4] ^ 8) << 4 (i = 0..3). Pinned by a round trip and by comparing the
elements it encodes with ``task1_ref.unpack_int4`` of the original.
"""

from __future__ import annotations

import numpy as np


def nibbles(w_q4: np.ndarray) -> np.ndarray:
    """[..., K/2] uint8 (reference packing) -> [..., K] element values 0..15."""
    b = np.asarray(w_q4, dtype=np.uint8)
    u = np.empty(b.shape[:-1] + (b.shape[-1] * 2,), dtype=np.uint8)
    u[..., 0::2] = b & 0xF
    u[..., 1::2] = b >> 4
    return u


def to_mfma(w_q4: np.ndarray) -> np.ndarray:
    u = nibbles(w_q4)
    runs = u.reshape(u.shape[:-1] + (-1, 8)) ^ 8
    out = (runs[..., 0:4] | (runs[..., 4:8] << 4)).astype(np.uint8)
    return out.reshape(np.asarray(w_q4).shape)


def from_mfma(w_mfma: np.ndarray) -> np.ndarray:
    b = np.asarray(w_mfma, dtype=np.uint8)
    runs = b.reshape(b.shape[:-1] + (-1, 4))
    lo = (runs & 0xF) ^ 8          # elements 0..3 of the run
    hi = (runs >> 4) ^ 8           # elements 4..7
    u = np.concatenate([lo, hi], axis=-1).reshape(b.shape[:-1] + (-1,))
    return (u[..., 0::2] | (u[..., 1::2] << 4)).astype(np.uint8)
