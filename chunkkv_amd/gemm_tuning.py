"""Library GEMM selection for the model's projections (PyTorch-ROCm TunableOp).

The model's GEMMs stay on PyTorch-ROCm (hipBLASLt / rocBLAS). Their default heuristic choice is
not always the fastest kernel at the prefill shapes of a blend request (8256 rows at layers 0-1,
~3000 at the others), so the choice is tuned once, offline, with TunableOp's own benchmark and
the resulting table is committed (``tuning/gemm_bf16_mi355x.csv``; validators: torch, HIP,
hipBLASLt, rocBLAS versions and the gfx950 target). ``use_tuned_gemms()`` makes torch pick from
that table and never tune at run time; a table whose validators do not match the running stack
is ignored by torch, and shapes missing from it keep the default choice. Precision is unchanged:
every candidate computes the same bf16 GEMM.

``python -m chunkkv_amd.gemm_tuning`` regenerates the table on an MI355X (a few minutes).
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import torch

TABLE = Path(__file__).resolve().parent / "tuning" / "gemm_bf16_mi355x.csv"


def use_tuned_gemms(table: Path = TABLE, scratch: str | None = None) -> bool:
    """Enable TunableOp in lookup-only mode with the committed table. Returns False (nothing
    changed) when the table is missing. `scratch` receives the file torch rewrites at exit."""
    if not table.exists():
        return False
    t = torch.cuda.tunable
    t.enable(True)
    t.tuning_enable(False)
    t.record_untuned_enable(False)
    t.set_filename(scratch or os.path.join(os.environ.get("TMPDIR", "/tmp"), "ckv_tunableop_results.csv"))
    return bool(t.read_file(str(table)))


def tune(out: Path = TABLE) -> None:
    """Tune the GEMM shapes of the 8k blend request (prefill, chunk prefills, last-token logits)
    and of greedy decode on a random-init Qwen2.5-7B architecture, for HipEngine (stacked q|k|v
    and gate|up projections) and for the reference op sequence (TorchOpsEngine, the model's own
    projections), so both run from tuned entries; write the table to `out`."""
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    import bench  # the workload definitions (request shape, model) live with the benchmark
    from chunkkv_amd.baseline import TorchOpsEngine
    from chunkkv_amd.engine import HipEngine
    from chunkkv_amd.types import BlendConfig

    t = torch.cuda.tunable
    t.enable(True)
    t.tuning_enable(True)
    t.set_filename(str(out))
    dev = torch.device("cuda:0")
    model = bench.random_qwen25_7b(dev)
    eng = HipEngine(model, bench._Tok())
    eng.decode_graphs = False  # tuning benchmarks cannot run inside a graph capture
    gen = torch.Generator().manual_seed(7)
    vocab = model.config.vocab_size
    pool = []
    for _ in range(bench.N_CHUNKS):
        toks = torch.randint(0, vocab, (bench.CHUNK_LEN,), generator=gen).tolist()
        pool.append((toks, eng.prefill(toks).chunk(0, bench.CHUNK_LEN)))
    tokens, placements = [], []
    for c in torch.randperm(len(pool), generator=gen).tolist():
        placements.append(bench.Place(pool[c][1], len(tokens)))
        tokens += pool[c][0]
    tokens += torch.randint(0, vocab, (bench.TAIL + bench.QUERY,), generator=gen).tolist()
    cfg = BlendConfig(recompute_ratio=bench.RATIO, n_sink=bench.N_SINK)
    res = eng.prefill(tokens, placements, cfg)
    TorchOpsEngine(model, bench._Tok()).prefill(tokens, placements, cfg)
    eng.last_logprobs(res)
    eng.eos = set()
    eng.generate(res, 2)
    torch.cuda.synchronize()
    t.tuning_enable(False)


if __name__ == "__main__":
    target = Path(sys.argv[1]) if len(sys.argv) > 1 else TABLE
    tune(target)
    print(f"tuned GEMM table -> {target}", flush=True)
