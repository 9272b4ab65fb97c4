"""Write tests/golden/projector_ref.safetensors with the reference's own Projector.save.

Run in the build container only (it imports the reference from /root/reference, which is absent on
GPU machines; the file it writes is what travels):

    python tests/golden/make_projector.py

The maps are tests/golden/c1.py's projector_tensors() (fp32; save() casts the [d_out, d_in + 1] map with
the bias as its last column to bf16, code/kva/kva.py:188-193), split c1.PROJ_SPLIT, metadata c1.PROJ_META.
The tests read this file with the oracle's and the product's Projector.load, compare the tensors bit
for bit with the cast of the same maps, and compare the bytes the product's save() writes for the same
maps and metadata with this file's.
"""
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
sys.path.insert(0, "/root/reference/code")

import c1  # noqa: E402


def main():
    from kva.kva import Projector
    maps = c1.projector_tensors()
    p = Projector(c1.PROJ_SPLIT, {L: w for L, (w, _) in maps.items()}, {L: b for L, (_, b) in maps.items()})
    p.save(c1.PROJ_FIXTURE, c1.PROJ_META)
    print(f"wrote {c1.PROJ_FIXTURE} ({c1.PROJ_FIXTURE.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
