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

tests/golden/finish_c1_arms.npz (same workload, the finish() branches the fixture above leaves open):
  4. fill 'none' with the 18 exact rows (only the rows reach the late layers; code/kva/kva.py:406-411);
  5. the exact arm with oracle_tap (code/kva/kva.py:310-316), then fill 'oracle' from the kept true inputs.

tests/golden/finish_q35.npz (the tiny Qwen3.5-style hybrid of tests/golden/q35.py, fp32 on the CPU):
  6. Qwen35.reads (code/kva/model.py:558-571) of every late layer on a held-out document -- GDN layers'
     pre-conv q / k / v and [b | a], the attention layer's k-normed K and V -- for the true inputs, a map's
     prediction and h_S itself, and fit_sweep's per-layer read cosine (code/scripts/fit_sweep.py:307-313);
  7. finish() with fill_by_type {'attention': 'proj', 'gdn': 'identity'} and st corrections (fill_store);
     the same arm without st (fill_store), then with st reusing that fill (fill_reuse); keep_cache=False;
     the by-type arm with 6 exact rows; the kvexact arm {'attention': 'oracle', 'gdn': 'proj'}.

    python tests/golden/make_golden.py [c1] [c1_arms] [q35]      (default: all three)
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
import q35  # noqa: E402


def fit_sweep_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("fit_sweep", REF_CODE / "scripts" / "fit_sweep.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def write_c1():
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


def write_c1_arms():
    from kva import model as M
    from kva.kva import Arm, finish, oracle_tap, run_lower
    torch.set_num_threads(8)
    with tempfile.TemporaryDirectory() as tmp:
        m = M.load(c1.write_checkpoint(Path(tmp) / "c1"), dtype=torch.float32)
        S, H = c1.SPLIT, m.hidden
        ids = c1.prompt_ids()
        n = ids.shape[0]
        P = n - c1.TAIL
        out = {}
        u_d, u_h, u_v = c1.probes(102, 64), c1.probes(100, H), c1.probes(103, 1024, 4)
        with torch.no_grad():
            hs, lower = run_lower(m, ids, {S})
            row_inputs = {}
            lg, cache, P1 = finish(m, ids, hs[S], lower, Arm("none", split=S, tail=c1.TAIL, fill="none"), c1.KEEP,
                                   exact_rows=c1.exact_rows(), row_inputs=row_inputs)
            rows = c1.exact_rows()
            out.update(none_P=np.array(P1), none_logits_u=(lg.double() @ u_v).numpy(),
                       none_argmax=lg.argmax(-1).numpy())
            for i in range(S, m.n_layers):
                c = cache[i]
                out[f"none_n_{i}"] = np.array(c["n"])
                for part in ("k", "v"):                   # slots: the exact rows, then the tail
                    out[f"none_{part}_u_{i}"] = (c[part].double() @ u_d).numpy()
                out[f"none_hr_u_{i}"] = (row_inputs[i].double() @ u_h).numpy()
            store = {}
            exact, ecache, _ = finish(m, ids, hs[S], lower, Arm("exact", split=S), c1.KEEP,
                                      hook=oracle_tap(store, S, P))
            lg, cache, P2 = finish(m, ids, hs[S], lower, Arm("oracle", split=S, tail=c1.TAIL, fill="oracle"), c1.KEEP,
                                   oracle=store)
            out.update(exact_logits_u=(exact.double() @ u_v).numpy(), oracle_P=np.array(P2),
                       oracle_logits_u=(lg.double() @ u_v).numpy(), oracle_argmax=lg.argmax(-1).numpy())
            for i in range(S, m.n_layers):
                out[f"oracle_in_u_{i}"] = (store[i].double() @ u_h).numpy()
                for part in ("k", "v"):
                    out[f"oracle_{part}_u_{i}"] = (cache[i][part].double() @ u_d).numpy()
                    out[f"exact_{part}_u_{i}"] = (ecache[i][part].double() @ u_d).numpy()
        out["rows"] = rows.numpy()
    path = HERE / "finish_c1_arms.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes, {len(out)} arrays)")


def write_q35():
    import torch.nn.functional as F
    from kva import model as M
    from kva.kva import Arm, Projector, finish, oracle_tap, run_lower
    torch.set_num_threads(8)
    with tempfile.TemporaryDirectory() as tmp:
        m = M.load(q35.write_checkpoint(Path(tmp) / "q35"), dtype=torch.float32)
        S, types = q35.SPLIT, m.layer_types
        maps, st = q35.maps(), q35.st()
        proj = Projector(S, {i: w for i, (w, _) in maps.items()}, {i: b for i, (_, b) in maps.items()})
        u_v = q35.probes(105, q35.VOCAB, 4)
        out = {}
        with torch.no_grad():
            got = {}
            m.forward_exact(q35.held_ids(), hook=lambda i, h: got.__setitem__(i, h) if i != "final" and i >= S
                            else None)
            for i in range(S, m.n_layers):
                true = m.reads(i, got[i])
                pred = m.reads(i, F.linear(got[S], maps[i][0], maps[i][1]))
                ident = m.reads(i, got[S])
                out.update(q35.read_arrays(f"true_{i}", true))
                out.update(q35.read_arrays(f"pred_{i}", pred))
                out[f"score_proj_{i}"] = np.array(q35.cosine_score(pred, true))
                out[f"score_identity_{i}"] = np.array(q35.cosine_score(ident, true))
            ids = q35.prompt_ids()
            hs, lower = run_lower(m, ids, {S})
            by_type = dict(split=S, tail=q35.TAIL, fill="by_type", fill_by_type={"attention": "proj", "gdn": "identity"},
                           projector=proj)
            runs = {}
            sa = {}
            runs["st"] = finish(m, ids, hs[S], lower, Arm("kva+st", st=st, **by_type), q35.KEEP, fill_store=sa)
            out.update(q35.cache_arrays("st_store", sa, runs["st"][2], types))
            sb = {}
            runs["base"] = finish(m, ids, hs[S], lower, Arm("kva", **by_type), q35.KEEP, fill_store=sb)
            runs["reuse"] = finish(m, ids, hs[S], lower, Arm("kva+st", st=st, **by_type), q35.KEEP, fill_reuse=sb)
            runs["nokeep"] = finish(m, ids, hs[S], lower, Arm("kva+st", st=st, **by_type), q35.KEEP, keep_cache=False)
            row_inputs = {}
            runs["exact"] = finish(m, ids, hs[S], lower, Arm("kva", **by_type), q35.KEEP, exact_rows=q35.exact_rows(),
                                   row_inputs=row_inputs)
            store = {}
            P = ids.shape[0] - q35.TAIL
            finish(m, ids, hs[S], lower, Arm("exact", split=S), q35.KEEP, hook=oracle_tap(store, S, P))
            runs["kvexact"] = finish(m, ids, hs[S], lower,
                                     Arm("kvexact", split=S, tail=q35.TAIL, fill="by_type", projector=proj,
                                         fill_by_type={"attention": "oracle", "gdn": "proj"}), q35.KEEP, oracle=store)
            for name, (lg, cache, P) in runs.items():
                out[f"{name}_P"] = np.array(P)
                out[f"{name}_logits_u"] = (lg.double() @ u_v).numpy()
                out[f"{name}_logits_last"] = lg[-1].double().numpy()
                out[f"{name}_argmax"] = lg.argmax(-1).numpy()
                out.update(q35.cache_arrays(name, cache, P, types))
            u_h = q35.probes(100, q35.H)
            for i in range(S, m.n_layers):
                out[f"exact_hr_u_{i}"] = (row_inputs[i].double() @ u_h).numpy()
    out = {k: v.astype(np.float32) if v.dtype == np.float64 and v.size > 1 else v for k, v in out.items()}
    np.savez_compressed(q35.FIXTURE, **out)
    print(f"wrote {q35.FIXTURE} ({q35.FIXTURE.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    writers = dict(c1=write_c1, c1_arms=write_c1_arms, q35=write_q35)
    for name in sys.argv[1:] or list(writers):
        writers[name]()
