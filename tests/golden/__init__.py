"""Golden vectors for the GDN decode / prefill path (see make_golden.py)."""
from pathlib import Path

HERE = Path(__file__).resolve().parent


def path(name: str) -> str:
    return str(HERE / name)
