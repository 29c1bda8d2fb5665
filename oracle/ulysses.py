"""CPU restatement of the Ulysses sequence <-> heads layouts.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

* ``qkv_send``            _qkv_send, src/taomate_hd/distributed/ulysses_layout.py:9-32
                          (element form: out[dest, p, t, l, d] = x[t, p*H + dest*L + l, d],
                          zero where dest*L + l >= H)
* ``qkv_send_token_major`` the same elements in the order [dest, t, p, l, d]
* ``qkv_send_reshape``    _merged_qkv_send_layout, distributed/ulysses.py:170-180
                          (view + permute; heads must divide evenly)
* ``all_to_all``          the collective: rank r receives chunk r of every rank's send
* ``qkv_receive``         outputs.movedim(0, 1).contiguous().view(3, U*T, L, D),
                          ulysses.py:209-211
* ``attention_receive``   _attention_receive, ulysses_layout.py:44-58
All arrays are numpy; values are moved, never computed, so results are exact.
Pinned by tests/test_oracle.py: the element form equals the reshape form
whenever the heads divide evenly; sequence -> heads -> sequence over U
emulated ranks returns every rank's original rows; rank r's received heads
are heads r*L.. of every rank's tokens in rank order.
"""

from __future__ import annotations

import numpy as np


def local_heads(heads: int, world: int) -> int:
    return (heads + world - 1) // world


def qkv_send(x: np.ndarray, heads: int, dim: int, world: int) -> np.ndarray:
    """Merged projection ``x [T, 3*H*D]`` -> ``[U, 3, T, L, D]`` (ulysses_layout.py:9-32)."""
    tokens = x.shape[0]
    local = local_heads(heads, world)
    src = x.reshape(tokens, 3, heads, dim)
    out = np.zeros((world, 3, tokens, local, dim), dtype=x.dtype)
    for dest in range(world):
        for l in range(local):
            head = dest * local + l
            if head < heads:
                out[dest, :, :, l, :] = src[:, :, head, :].transpose(1, 0, 2)
    return out


def qkv_send_token_major(x: np.ndarray, heads: int, dim: int, world: int) -> np.ndarray:
    """The same elements as ``qkv_send`` in the order ``[U, T, 3, L, D]``."""
    return qkv_send(x, heads, dim, world).transpose(0, 2, 1, 3, 4).copy()


def qkv_send_reshape(x: np.ndarray, heads: int, dim: int, world: int) -> np.ndarray:
    """_merged_qkv_send_layout (ulysses.py:170-180): view then permute(2, 1, 0, 3, 4)."""
    if heads % world:
        raise ValueError("the reshape form needs heads divisible by the world size")
    tokens = x.shape[0]
    return x.reshape(tokens, 3, world, heads // world, dim).transpose(2, 1, 0, 3, 4).copy()


def all_to_all(sends: list[np.ndarray]) -> list[np.ndarray]:
    """``sends[s]`` is rank s's buffer with a leading [U] destination axis;
    rank r receives ``[U(source), ...]`` with chunk r of every rank."""
    world = len(sends)
    return [np.stack([sends[s][r] for s in range(world)]) for r in range(world)]


def qkv_receive(received: np.ndarray) -> np.ndarray:
    """``[U, 3, T, L, D]`` -> ``[3, U*T, L, D]`` (ulysses.py:209-211)."""
    world, _, tokens, local, dim = received.shape
    return received.transpose(1, 0, 2, 3, 4).reshape(3, world * tokens, local, dim).copy()


def attention_receive(received: np.ndarray, heads: int) -> np.ndarray:
    """``[U, T, L, D]`` (source rank s holds heads s*L..) -> ``[T, H, D]``
    (ulysses_layout.py:44-58; padded heads dropped)."""
    world, tokens, local, dim = received.shape
    out = np.empty((tokens, heads, dim), dtype=received.dtype)
    for head in range(heads):
        out[:, head, :] = received[head // local, :, head % local, :]
    return out
