"""Seeded inputs shared by the tests: paged caches in the three layouts, raw-bit views.

The literal shapes are the reference tests' (core/tests/test_gather_kernel.py:18-20,67-69,91-102):
seven blocks of four slots, three head slots, three layers, slots [5, -1, 17, 0, 27] with one
padding id, held heads [0, 2], capacity 8, d in {8, 6} (16-byte rows and not).
"""

from __future__ import annotations

import numpy as np
import torch

import oracle

NB, BS, H, L = 7, 4, 3, 3
SLOTS = [5, -1, 17, 0, 27]
HEADS = [0, 2]
CAPACITY = 8
LAYOUTS = ("kv_first", "blocks_first", "combined")
DTYPES = (torch.bfloat16, torch.float16, torch.float32, torch.float8_e4m3fn)
NP_BITS = {1: np.uint8, 2: np.uint16, 4: np.uint32}
TORCH_BITS = {1: torch.uint8, 2: torch.int16, 4: torch.int32}


def cache_shape(layout: str, nb: int, bs: int, h: int, d: int) -> tuple[int, ...]:
    return {
        "kv_first": (2, nb, bs, h, d),
        "blocks_first": (nb, 2, bs, h, d),
        "combined": (nb, h, bs, 2 * d),
    }[layout]


def caches(layout: str, d: int, dtype, n_layers: int = L, nb: int = NB, bs: int = BS, h: int = H,
           seed: int = 3) -> list[torch.Tensor]:
    """``n_layers`` CPU caches of N(0, 1) values (fp8: N(0, 1) / 0.05, saturated to e4m3's range)."""
    g = torch.Generator().manual_seed(seed)
    shape = cache_shape(layout, nb, bs, h, d)
    out = []
    for _ in range(n_layers):
        x = torch.randn(shape, generator=g)
        if dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
            x = (x / 0.05).clamp(-448, 448)
        out.append(x.to(dtype))
    return out


def bits(t: torch.Tensor) -> np.ndarray:
    """A tensor's raw bits as an unsigned numpy array (CPU)."""
    e = t.element_size()
    return t.detach().cpu().contiguous().view(TORCH_BITS[e]).numpy().view(NP_BITS[e])


def strides_of(t: torch.Tensor) -> tuple[int, int, int, int, int]:
    layout, _, _, d = oracle.recognise(t.shape)
    return oracle.layout_strides(layout, t.stride(), d)


def brute_gather(layers, slots, heads, capacity: int) -> np.ndarray:
    """The gather by its definition per layout, one row at a time, with numpy indexing by
    dimension (no strides): out[l, h, t, k, j] = the K (k=0) or V (k=1) element j of head slot
    heads[h] at slot max(slots[t], 0)."""
    layout, _, bs, d = oracle.recognise(layers[0].shape)
    e = layers[0].element_size()
    out = np.zeros((len(layers), len(heads), capacity, 2, d), dtype=NP_BITS[e])
    for li, t in enumerate(layers):
        a = bits(t)
        for hi, head in enumerate(heads):
            for ti, s in enumerate(slots):
                s = max(int(s), 0)
                b, o = divmod(s, bs)
                for k in range(2):
                    if layout == "kv_first":
                        row = a[k, b, o, head, :]
                    elif layout == "blocks_first":
                        row = a[b, k, o, head, :]
                    else:
                        row = a[b, head, o, k * d:(k + 1) * d]
                    out[li, hi, ti, k] = row
    return out


def random_case(seed: int) -> dict:
    """One seeded draw over what a caller may pass: any of the three layouts, element type, head
    dim (16-byte rows and not), block size (powers of two and not), head count, a held-head list
    in any order, 1 to 200 slots (about one in ten padding), spare capacity, and the cache as a
    contiguous tensor, a head-sliced view of a wider one, or (combined) the reference's permuted
    [nb, bs, h, 2d] build. ``base`` holds the CPU tensors the caches are views of; ``view`` turns
    one (or its device copy) into the cache, so that a device cache keeps the same strides."""
    rng = np.random.default_rng(seed)
    layout = LAYOUTS[int(rng.integers(len(LAYOUTS)))]
    dtype = DTYPES[int(rng.integers(len(DTYPES)))]
    d = int(rng.choice([2, 4, 6, 8, 16, 24, 64, 128]))
    bs = int(rng.choice([1, 2, 3, 4, 5, 7, 16]))
    h = int(rng.integers(1, 10))
    nb = int(rng.integers(1, 41))
    n_layers = int(rng.integers(1, 4))
    heads = rng.permutation(h)[:int(rng.integers(1, h + 1))].tolist()
    n = int(rng.integers(1, min(nb * bs, 200) + 1))
    slots = rng.choice(nb * bs, size=n, replace=False).astype(np.int64)
    slots[rng.random(n) < 0.1] = -1
    kind = rng.choice(["contiguous", "head_slice", "permuted"] if layout == "combined"
                      else ["contiguous", "head_slice"])
    g = torch.Generator().manual_seed(seed)
    wide = h + 1 if kind == "head_slice" else h
    if kind == "permuted":
        shape = (nb, bs, h, 2 * d)

        def view(t):
            return t.permute(0, 2, 1, 3)
    else:
        shape = cache_shape(layout, nb, bs, wide, d)
        hdim = 1 if layout == "combined" else 3

        def view(t):
            return t.narrow(hdim, wide - h, h)
    base = []
    for _ in range(n_layers):
        x = torch.randn(shape, generator=g)
        if dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
            x = (x / 0.05).clamp(-448, 448)
        base.append(x.to(dtype))
    return dict(seed=seed, layout=layout, dtype=dtype, d=d, bs=bs, h=h, nb=nb, heads=heads,
                slots=slots, cap=n + int(rng.integers(0, 5)), kind=str(kind), base=base,
                view=view, rng=rng)


def brute_scatter(layers, slots, heads, rows) -> list[np.ndarray]:
    """The scatter by its definition per layout, on raw-bit copies of ``layers``: for each listed
    slot s >= 0 at position t, the K (k=0) or V (k=1) half-row of head slot heads[h] at s becomes
    rows[l, h, t, k]; everything else keeps its bits. Returns the new bits, one array a layer."""
    layout, _, bs, d = oracle.recognise(layers[0].shape)
    out = []
    for li, t in enumerate(layers):
        a = bits(t).copy()
        for hi, head in enumerate(heads):
            for ti, s in enumerate(slots):
                if s < 0:
                    continue
                b, o = divmod(int(s), bs)
                for k in range(2):
                    if layout == "kv_first":
                        a[k, b, o, head, :] = rows[li, hi, ti, k]
                    elif layout == "blocks_first":
                        a[b, k, o, head, :] = rows[li, hi, ti, k]
                    else:
                        a[b, head, o, k * d:(k + 1) * d] = rows[li, hi, ti, k]
        out.append(a)
    return out


SPECIAL_N = 1 << 16


def special_members() -> dict[int, np.ndarray]:
    """bf16 members (raw bits) that reach the sum's special cases, SPECIAL_N elements each.

    0: every bf16 bit pattern once: zeros of both signs, subnormals, the largest finite values,
       infinities and NaNs of both signs;
    1: the same patterns rotated, so that inf meets -inf, NaN meets numbers and large values of
       one sign meet (an fp32 sum past bf16's range rounds to infinity);
    2: uniform random bits;
    3: half a bf16 unit in the last place of member 0's value, with its sign (zero where that
       is not a normal bf16), so that member 0 + member 3 is an exact tie for the rounding.
    """
    every = np.arange(SPECIAL_N, dtype=np.uint32).astype(np.uint16)
    expo = (every.astype(np.int32) >> 7) & 0xFF
    half_ulp = np.where((expo > 8) & (expo < 255),
                        ((expo - 8) << 7) | (every.astype(np.int32) & 0x8000), 0).astype(np.uint16)
    rng = np.random.default_rng(77)
    return {0: every, 1: np.roll(every, 40961),
            2: rng.integers(0, 1 << 16, size=SPECIAL_N, dtype=np.uint16), 3: half_ulp}


def bf16_tensor(raw: np.ndarray) -> torch.Tensor:
    """A CPU bf16 tensor holding the raw bits ``raw`` (uint16)."""
    return torch.from_numpy(np.ascontiguousarray(raw).view(np.int16)).view(torch.bfloat16)


def fp8_scaled_layers(n_layers: int, shape, seed: int, device: str = "cuda"):
    """C3's fp8-e4m3 cache: layer l holds fp8(N(0, 1) / s_l) with per-layer scales s_l ~ U(0.01,
    0.1) (numpy rng ``seed``), saturated to e4m3's +-448 as a cast from a wider type saturates.
    Layer 0's first 256 bytes are then overwritten with every byte code 0..255, so the NaN codes
    (0x7F, 0xFF), the saturation codes and the subnormals are all among the bytes moved.

    Returns (layers, scales) with scales a float32 numpy array [n_layers]."""
    scales = np.random.default_rng(seed).uniform(0.01, 0.1, n_layers).astype(np.float32)
    g = torch.Generator(device=device).manual_seed(seed)
    out = []
    for s in scales.tolist():
        x = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
        out.append((x / s).clamp_(-448, 448).to(torch.float8_e4m3fn))
    out[0].view(torch.uint8).view(-1)[:256] = torch.arange(256, dtype=torch.uint8,
                                                           device=device)
    return out, scales
