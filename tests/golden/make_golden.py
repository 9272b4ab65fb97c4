"""Write tests/golden/finish_c1.npz from the reference implementation itself.

Run in the build container only (it reads the reference from /root/reference, which is absent on GPU
machines; the fixture it writes is what travels):

    python tests/golden/make_golden.py

What it runs, on the tiny Llama-style workload of tests/golden/c1.py, in fp32 on the CPU:
  1. the capture of fit_sweep (code/scripts/fit_sweep.py:62-166: accumulators, capture_hook over
     Model.forward_exact, split_state) on the 4096-token calibration document, split 5, and on two
     short documents (whose shifts are the first document's means, not the overall means);
  2. RidgeFit.layer (code/kva/ridge.py:77-105) for layers 5..7 at lambda 1e-2 -> a Projector
     (code/kva/kva.py:137-159);
  3. run_lower + finish (code/kva/kva.py:282-300, 319-460) on the 2048-token prompt with tail 256:
     the ridgefill arm (fill 'proj'), the identity arm, and the ridgefill arm with 18 exact rows
     (layer_rows, row_inputs recorded).
The fixture keeps the capture sums, the maps, the filled K / V caches, the exact rows' late-layer
inputs and the tail logits, large tensors as projections onto fixed probe vectors (tests/golden/c1.py).
"""
import sys
import tempfile
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REF_CODE = Path("/root/reference/code")
sys.path.insert(0, str(HERE))
sys.path.insert(0, str(REF_CODE))

import c1  # noqa: E402


def fit_sweep_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("fit_sweep", REF_CODE / "scripts" / "fit_sweep.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main():
    from kva import model as M
    from kva.kva import Arm, Projector, finish, run_lower
    from kva.ridge import RidgeFit
    torch.set_num_threads(8)
    fs = fit_sweep_module()
    with tempfile.TemporaryDirectory() as tmp:
        path = c1.write_checkpoint(Path(tmp) / "c1")
        m = M.load(path, dtype=torch.float32)
        L, H, S = m.n_layers, m.hidden, c1.SPLIT

        def capture(docs):
            acc = fs.accumulators([S], L, H)
            xs = {}
            hook = fs.capture_hook(acc, xs)
            for doc in docs:
                xs.clear()
                m.forward_exact(doc, hook=hook)
                acc["n"] += doc.shape[0]
            return fs.split_state(acc, S, L, H)

        with torch.no_grad():
            state = capture([c1.calibration_ids()])
            state2 = capture(c1.two_documents())
            fit = RidgeFit(state)
            maps = {i: fit.layer(i, (c1.LAM,))[c1.LAM] for i in range(S, L)}
            proj = Projector(S, {i: w for i, (w, _) in maps.items()}, {i: b for i, (_, b) in maps.items()})
            ids = c1.prompt_ids()
            hs, lower = run_lower(m, ids, {S})
            runs = {}
            lg, cache, P = finish(m, ids, hs[S], lower, Arm("kva", split=S, tail=c1.TAIL, fill="proj",
                                                            projector=proj), c1.KEEP)
            runs["proj"] = (lg, cache, P, None)
            lg, cache, P = finish(m, ids, hs[S], lower, Arm("noproj", split=S, tail=c1.TAIL, fill="identity"),
                                  c1.KEEP)
            runs["identity"] = (lg, cache, P, None)
            row_inputs = {}
            lg, cache, P = finish(m, ids, hs[S], lower, Arm("kva", split=S, tail=c1.TAIL, fill="proj",
                                                            projector=proj), c1.KEEP,
                                  exact_rows=c1.exact_rows(), row_inputs=row_inputs)
            runs["exact"] = (lg, cache, P, row_inputs)
    out = c1.summarise(state, state2, maps, runs)
    out["h_split_u"] = (hs[S].double() @ c1.probes(100, H)).numpy()
    np.savez_compressed(c1.FIXTURE, **out)
    print(f"wrote {c1.FIXTURE} ({c1.FIXTURE.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
