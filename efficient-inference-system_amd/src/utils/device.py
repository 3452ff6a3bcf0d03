"""Device pick, as src/utils/device.py:3-4 of the reference."""
import torch


def get_device() -> str:
    return "cuda" if torch.cuda.is_available() else "cpu"
