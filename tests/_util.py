"""Helpers shared by the tests."""
import sys


def log_case(msg):
    """Print and flush what a GPU step is about to run, so a failure names its case."""
    print(f'[case] {msg}', flush=True)
    sys.stdout.flush()


def rel_err(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


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
