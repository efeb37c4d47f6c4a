"""Copy a few lines of the reference's RoPE ROM text files into tests/golden/.

    python tests/golden/make_memh_slices.py [/path/to/reference]

rtl/compute/rope_{cos,sin}_rom.memh hold 2048 positions x 32 Q16.16 words,
one 8-digit hexadecimal word per line, written by EX:199-217 write_hex_memh
(EX:656-681).  The 32 lines of each position in POSITIONS are kept verbatim:
they pin the memh reader and writer of golden_trace.py byte for byte (the
decoded values are also in rope_rom.npz).  Only the data files are read.
"""
from __future__ import annotations

import os
import sys

OUT = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
POSITIONS = (0, 1, 93, 1021, 2047)


def main() -> None:
    for kind in ("cos", "sin"):
        with open(os.path.join(REF, "rtl", "compute", f"rope_{kind}_rom.memh")) as fh:
            lines = fh.read().split("\n")
        keep = [lines[p * 32 + d] for p in POSITIONS for d in range(32)]
        with open(os.path.join(OUT, f"rope_{kind}_rom_slice.memh"), "w") as fh:
            fh.write("\n".join(keep) + "\n")


if __name__ == "__main__":
    main()
