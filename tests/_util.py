"""Helpers shared by the tests."""
import sys


def log_case(msg):
    """Print and flush what a GPU step is about to run, so a failure names its case."""
    print(f'[case] {msg}', flush=True)
    sys.stdout.flush()


def rel_err(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def wtile_index(rows, cols):
    """Flat offset of element (n, k) of a bf16 weight [rows, cols] in the library's WTILE layout
    (NOISE_LAYOUT_WTILE of include/noise_hip.h), built from the header's forward description: block (g, s) at
    (g * cols / 32 + s) * 512 holds columns 32 s .. 32 s + 31 of the rows with tiled index i = 16 g + r, row r of
    the block being weight row (i - i % 64) + (r // 4) * 16 + ((i % 64) // 16) * 4 + r % 4, its 16-byte chunk c
    at c ^ ((r // 2) % 4). The weight row of each tiled index is inverted by a scatter."""
    import torch
    i = torch.arange(rows)
    r = i % 16
    row_of = (i - i % 64) + (r // 4) * 16 + ((i % 64) // 16) * 4 + r % 4
    tiled_of = torch.empty_like(i)
    tiled_of[row_of] = i
    assert torch.equal(torch.sort(row_of).values, i), 'not a permutation'
    ti = tiled_of[:, None]
    tr = ti % 16
    k = torch.arange(cols)[None, :]
    return ((ti // 16) * (cols // 32) + k // 32) * 512 + 32 * tr + 8 * (((k % 32) // 8) ^ ((tr // 2) % 4)) + k % 8


def tile16_index(rows, cols):
    """Flat offset of element (r, c) of a bf16 [rows, cols] matrix in the library's TILE16 layout
    (NOISE_LAYOUT_TILE16 of include/noise_hip.h): 1 KiB tiles of 16 rows x 32 columns, row groups outermost;
    inside a tile, 16-byte unit p = 4 (r % 16) + (((c % 32) // 8) ^ (((r % 16) // 2) % 4))."""
    import torch
    r = torch.arange(rows)[:, None]
    c = torch.arange(cols)[None, :]
    rr = r % 16
    p = 4 * rr + (((c % 32) // 8) ^ ((rr // 2) % 4))
    return (r // 16) * 16 * cols + (c // 32) * 512 + 8 * p + c % 8
