"""Helpers shared by the tests."""
import sys


def log_case(msg):
    """Print and flush what a GPU step is about to run, so a failure names its case."""
    print(f'[case] {msg}', flush=True)
    sys.stdout.flush()


def rel_err(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))
