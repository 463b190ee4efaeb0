"""Autotuner of the per-M dispatch table (run on the GPU the table is for).

The counterpart of the reference's bench/tune_configs.py, which times Triton
block-size candidates per M and writes vLLM's per-device config JSON.  Here
the candidates are the dispatch choices of struct w4a16_moe_tuning (GEMV-only
vs. GEMV + MFMA split, the split threshold, GEMV token rows per pass); each is
timed on the full-size synthetic layer with HIP-graph replays over rotating
routing sets (so the weights come from HBM, not the Infinity Cache), under
both uniform routing and skewed routing (a per-expert logit bias, which gives
some experts many more pairs), and its output is checked against the
built-in choice before it can win.  A candidate's score is the sum of its
two times relative to the built-in choice's.  The best candidate is then
re-timed against the built-in choice in CONFIRM_ROUNDS alternating rounds and
replaces it only when the median score improves by more than MIN_GAIN
(identical dispatches differ by a few percent between graph timings).

    python gb10-laguna-s-2.1-w4a16-moe_amd/tune.py [--ms 1,2,4,...] [--out DIR]
           [--E 256 --N 1024 --K 3072 --group 32 --topk 10] [--report FILE]

writes DIR/<tuning.config_name(...)> (default DIR: the package's configs/).
"""

from __future__ import annotations

import argparse
import importlib
import importlib.util
import json
import math
import sys
import time
from pathlib import Path

MALL_BYTES = 256 * 2**20
MIN_GAIN = 0.03
CONFIRM_ROUNDS = 3
DEFAULT_MS = (1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128, 256, 512, 1024, 2048, 4096)
PKG_NAME = "w4a16_moe_amd"


def _pkg():
    """The package this file belongs to (imported by path when run as a script)."""
    if __package__:
        return sys.modules[__package__]
    mod = sys.modules.get(PKG_NAME)
    if mod is not None:
        return mod
    d = Path(__file__).resolve().parent
    spec = importlib.util.spec_from_file_location(PKG_NAME, d / "__init__.py",
                                                  submodule_search_locations=[str(d)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[PKG_NAME] = mod
    spec.loader.exec_module(mod)
    return mod


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def effective(M: int, N: int, K: int, t, builtin_tile: int = 192) -> tuple:
    """What a tuning does at M: the GEMV-only or the split dispatch
    (builtin_tile: the MFMA tile height mfma_tile_m = 0 selects at M)."""
    if M <= t.gemv_only_max_m or N % 256 or K % 256:
        fused = M <= (t.w2_fused_max_m or 4)
        return ("gemv", t.gemv_tokens_per_pass, t.gemv_units_per_wg, t.gemv_lanes_per_row,
                fused)
    return ("split", t.gemv_max_tokens,
            t.gemv_tokens_per_pass if t.gemv_max_tokens else 0,
            t.gemv_units_per_wg if t.gemv_max_tokens else 0,
            t.gemv_lanes_per_row if t.gemv_max_tokens else 0,
            t.mfma_tile_m or builtin_tile, t.mfma_row_tiles)


def candidates(M: int, N: int, K: int, Tuning, always: int, base=None):
    """Every distinct dispatch choice worth timing at M, the built-in one
    (`base`, the library's own choice for M) first; slow candidates are pruned
    against it."""
    out = [base if base is not None else Tuning()]
    for tc in (0, 1, 2, 4):
        if tc == 1 and M > 4:
            continue
        out += [Tuning(always, 4, tc, 0, upw) for upw in (0, 1, 2, 4)]
        if tc in (0, 1, 2):
            out += [Tuning(always, 4, tc, 0, 0, lpr) for lpr in (8, 32)]
    if 1 < M <= 16:  # w2 with the top-k sum as one kernel
        out += [Tuning(always, 4, tc, 0, 0, 0, M) for tc in (0, 2, 4)]
    if M > 1 and N % 256 == 0 and K % 256 == 0:
        for thr in (0, 2, 4, 8, 15):
            for tc in (0, 2, 4):
                out.append(Tuning(0, thr, tc, 0))
        out += [Tuning(0, 4, 0, 0, upw) for upw in (1, 2, 4)]
        # MFMA token tiles of at most 64 or 128 slots (more, smaller tiles)
        out += [Tuning(0, thr, 0, tm) for thr in (0, 4) for tm in (64, 128, 192)]
    builtin_tile = base.mfma_tile_m if base is not None and base.mfma_tile_m else 192
    seen, uniq = set(), []
    for t in out:
        key = effective(M, N, K, t, builtin_tile)
        if key not in seen:
            seen.add(key)
            uniq.append(t)
    return uniq


class _Bench:
    def __init__(self, pkg, shape, weights, M, dev, seed_base=0, skewed=False):
        import torch

        synth = importlib.import_module(pkg.__name__ + ".synth")
        self.pkg, self.shape, self.M, self.dev = pkg, shape, M, dev
        self.w = weights
        expect = min(shape.E, M * shape.topk) * shape.bytes_per_expert
        n_sets = min(32, max(4, math.ceil(2 * MALL_BYTES / expect)))
        self.sets = []
        for i in range(n_sets):
            x = synth.make_hidden(M, shape.K, dev, seed=seed_base + i)
            tw, ti = synth.make_routing(M, shape.E, shape.topk, dev, seed=seed_base + i,
                                        skewed=skewed, bias_seed=0)
            self.sets.append((x, tw, ti))
        torch.cuda.synchronize()

    def call(self, i, tuning):
        x, tw, ti = self.sets[i]
        w13, w2, s13, s2 = self.w
        return self.pkg.fused_experts_w4a16(x, w13, w2, s13, s2, tw, ti, self.shape.group,
                                            tuning=tuning)

    def quick_us(self, tuning):
        """One eager pass over the sets (for pruning)."""
        import torch

        self.call(0, tuning)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(len(self.sets)):
            self.call(i, tuning)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e6 / len(self.sets)

    def graph_us(self, tuning, min_ms=20.0):
        import torch

        n = len(self.sets)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for i in range(n):
                self.call(i, tuning)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                self.call(i, tuning)
        g.replay()
        torch.cuda.synchronize()
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        g.replay()
        en.record()
        torch.cuda.synchronize()
        once = st.elapsed_time(en)
        reps = max(2, min(200, int(min_ms / max(once, 1e-3))))
        st.record()
        for _ in range(reps):
            g.replay()
        en.record()
        torch.cuda.synchronize()
        return st.elapsed_time(en) * 1e3 / (reps * n)


def tune(ms, E, N, K, group, topk, seed=0, check_tol=5e-3):
    """Return ({M: best Tuning}, report rows)."""
    import torch

    pkg = _pkg()
    T = pkg.tuning
    dev = torch.device("cuda", torch.cuda.current_device())
    synth = importlib.import_module(pkg.__name__ + ".synth")
    shape = synth.LayerShape(E=E, topk=topk, K=K, N=N, group=group)
    weights = synth.make_weights(shape, dev, seed=seed)
    table, report = {}, []
    for M in ms:
        benches = {"uniform": _Bench(pkg, shape, weights, M, dev, seed_base=1000 * M),
                   "skewed": _Bench(pkg, shape, weights, M, dev, seed_base=1000 * M,
                                    skewed=True)}
        # the built-in choices for M, as explicit values
        base = T.Tuning.from_struct(pkg._lib.default_tuning(M, topk, E, N, K, group))
        refs = {k: b.call(0, base).float() for k, b in benches.items()}
        base_us = {k: b.graph_us(base) for k, b in benches.items()}
        base_q = {k: b.quick_us(base) for k, b in benches.items()}
        rows = []
        best = (2.0, base, dict(base_us))
        for cand in candidates(M, N, K, T.Tuning, T.ALWAYS, base)[1:]:
            for k, b in benches.items():
                out = b.call(0, cand).float()
                torch.cuda.synchronize()
                rel = (out - refs[k]).norm().item() / max(refs[k].norm().item(), 1e-30)
                if not rel <= check_tol:
                    raise RuntimeError(f"M={M} {k} {cand}: output differs from the built-in "
                                       f"choice (rel_l2 {rel:.3e})")
            q = sum(b.quick_us(cand) / base_q[k] for k, b in benches.items())
            if q > 4.0:  # twice the built-in time on average: not a contender
                rows.append({"tuning": cand.to_dict(), "quick_score": round(q, 3),
                             "pruned": True})
                continue
            us = {k: b.graph_us(cand) for k, b in benches.items()}
            score = sum(us[k] / base_us[k] for k in us)
            log(f"  M={M} {cand}: score {score:.3f}")
            rows.append({"tuning": cand.to_dict(), "score": round(score, 4),
                         "us": {k: round(v, 3) for k, v in us.items()}})
            if score < best[0]:
                best = (score, cand, us)
        confirmed = None
        if best[1] != base:
            scores = []
            for _ in range(CONFIRM_ROUNDS):
                b_us = {k: b.graph_us(base) for k, b in benches.items()}
                c_us = {k: b.graph_us(best[1]) for k, b in benches.items()}
                scores.append(sum(c_us[k] / b_us[k] for k in b_us))
            confirmed = sorted(scores)[len(scores) // 2]
            if confirmed > 2.0 * (1.0 - MIN_GAIN):
                best = (2.0, base, dict(base_us))
        table[M] = best[1]
        report.append({"M": M, "sets": {k: len(b.sets) for k, b in benches.items()},
                       "best": best[1].to_dict(), "best_score": round(best[0], 4),
                       "confirm_score": None if confirmed is None else round(confirmed, 4),
                       "best_us": {k: round(v, 3) for k, v in best[2].items()},
                       "builtin_us": {k: round(v, 3) for k, v in base_us.items()},
                       "candidates": rows})
        log(f"M={M:5d}: {best[1]} score {best[0]:.3f} (confirmed {confirmed}); uniform {best[2]['uniform']:.1f} us "
            f"(built-in {base_us['uniform']:.1f}), skewed {best[2]['skewed']:.1f} us "
            f"(built-in {base_us['skewed']:.1f})")
        del benches, refs
        pkg.w4a16_moe._WS_POOL.clear()  # the candidates' graphs are gone
        torch.cuda.empty_cache()
    return table, report


def main(argv=None) -> int:
    import torch

    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--ms", default=",".join(map(str, DEFAULT_MS)))
    ap.add_argument("--E", type=int, default=256)
    ap.add_argument("--N", type=int, default=1024)
    ap.add_argument("--K", type=int, default=3072)
    ap.add_argument("--group", type=int, default=32)
    ap.add_argument("--topk", type=int, default=10)
    ap.add_argument("--out", default=None, help="directory for the table JSON")
    ap.add_argument("--report", default=None, help="write every candidate's time here")
    ap.add_argument("--replace", action="store_true",
                    help="write only the tuned M (default: merge into an existing table)")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        log("tune.py needs the GPU the table is for")
        return 2
    pkg = _pkg()
    T = pkg.tuning
    ms = [int(v) for v in args.ms.split(",") if v]
    # time the built-in choices only: ignore any table already on disk
    import os

    os.environ["W4A16_MOE_TUNING"] = "default"
    table, report = tune(ms, args.E, args.N, args.K, args.group, args.topk)
    out_dir = Path(args.out) if args.out else T.CONFIG_DIR
    out_dir.mkdir(parents=True, exist_ok=True)
    path = out_dir / T.config_name(args.E, args.N, args.K, args.group, T.device_name())
    if path.exists() and not args.replace:
        # keep the entries of an existing table for the M not tuned now
        old = T.load_table(args.E, args.N, args.K, args.group, T.device_name(), out_dir) or {}
        table = {**{m: t for m, t in old.items() if m not in table}, **table}
    path.write_text(T.dump_table(table))
    log(f"wrote {path}")
    if args.report:
        Path(args.report).write_text(json.dumps({"device": T.device_name(), "E": args.E,
                                                 "N": args.N, "K": args.K, "group": args.group,
                                                 "topk": args.topk, "rows": report}, indent=1))
    print(json.dumps({"table": str(path), "entries": len(table)}))
    return 0


if __name__ == "__main__":
    sys.exit(main())
