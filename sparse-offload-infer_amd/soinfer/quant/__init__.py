"""Weight quantization and INT4 packing: the producer of every kernel's input bytes."""
from . import calibrate, formats, pack

__all__ = ["formats", "pack", "calibrate"]
