"""Per-op benchmark CLI: the reference's ``benchmarks/bench_<op>.py`` contract.

    python -m ezops.bench_ops <op> [-k hip,ref] [-w label,...] [--json PATH]
    python -m ezops.bench_ops <op> -h          # list the op's backends
    python -m ezops.bench_ops all              # every op below

For each workload (the reference bench's own list, then the decode path's
benchmark configurations) the harness does what the reference benches do
(benchmarks/bench_gemv.py:89-161, benchmarks/bench_reduce.py:87-150):

1. ``backend="ref"`` builds the op; its ``_ref_forward`` on the GPU gives the
   expected output, ``get_roofline()`` the algorithmic flops and bytes, and
   its latency is the 1.00x row;
2. per backend, untimed and in this order: one call checked with the op's
   ``check`` and an SQNR >= 28 dB, two more calls compared byte for byte
   (determinism), one call with the inputs compared byte for byte before and
   after (read-only; the KV caches that the fused ops write by design are
   excluded);
3. latency = ``bench_kernel`` (HIP graphs, a 1 GiB read flush before every
   call, the flush+call graph timed against the flush-only graph, median
   over 5 trials of 100 calls); speedup over ref and
   the sol-score = theoretical minimum time / latency, where the minimum is
   ``hardware.compute_sol`` of the MI355X profile (tf32 = fp32 MFMA peak,
   calibrated HBM read rate).

Output: the reference's two tables per workload (performance; SOL analysis)
and, with ``--json``, one record per (workload, backend).
"""

from __future__ import annotations

import argparse
import json
import math
import sys
from dataclasses import dataclass, field
from typing import Callable

import torch

from . import hardware, workloads
from .ops.utils.accuracy import SQNR_THRESHOLD_DB, bitwise_equal
from .registry import list_backends

WARMUP = 10
N_REPEAT = 100
N_TRIALS = 5


@dataclass
class Workload:
    """One benchmark case of an op.

    ``make(backend)`` builds the op; ``data(ref_op, device)`` returns
    ``(ref_args, kernel_args)`` (the same tensors except where the reference
    takes another layout, as GEMV's [K, N] weight); ``out`` are the argument
    positions the op writes its result into (None: the op returns it);
    ``mutable`` are positions the op also writes by design (KV caches);
    ``input_bytes(ref_op, args)`` is the fused-memory byte count of the SOL
    (default, as the reference benches: every argument that is not an
    output; ops that index into a cache count only the rows they read)."""

    label: str
    shape: str
    make: Callable
    data: Callable
    out: tuple | None = None
    mutable: tuple = ()
    input_bytes: Callable | None = None
    repeat: int = N_REPEAT


@dataclass
class OpBench:
    name: str          # registry name (``list_backends`` key)
    title: str
    workloads: list = field(default_factory=list)


def _same(ref_op, device):
    d = ref_op.gen_data(device=device)
    d = d if isinstance(d, tuple) else (d,)
    return d, d


# ---- GEMV (reference: benchmarks/bench_gemv.py:27-34, 100-110) --------------
def _gemv(N, K, label):
    from .ops.gemv import GemvOp

    def data(ref_op, device):
        torch.manual_seed(42)
        A = torch.randn(K, device=device).to(torch.bfloat16)
        B_nk = torch.randn(N, K, device=device).to(torch.bfloat16)
        C = torch.empty(N, dtype=torch.bfloat16, device=device)
        return (A, B_nk.T.contiguous(), C), (A, B_nk, C.clone())

    return Workload(label, f"A ({K},)  B ({N}, {K})  C ({N},)", lambda b: GemvOp(N, K, backend=b), data, out=(2,))


def _gemv_g():
    from .ops.gemv import GemvOp

    def data(ref_op, device):
        x, W = workloads.config_g(device)
        y = torch.empty(4096, dtype=torch.bfloat16, device=device)
        return (x, W.T.contiguous(), y), (x, W, y.clone())

    return Workload("config-G-4096x4096", "x (4096,)  W (4096, 4096)  y (4096,)",
                    lambda b: GemvOp(4096, 4096, backend=b), data, out=(2,))


# ---- row ops (reference: benchmarks/bench_{rmsnorm,softmax,reduce}.py) -----
def _rmsnorm(B, D, label, weighted=False, dtype=torch.float32):
    from .ops.rmsnorm import RmsNormOp

    return Workload(label, f"X ({B}, {D}) {str(dtype)[6:]}" + (" + weight" if weighted else ""),
                    lambda b: RmsNormOp(B, D, backend=b, dtype=dtype, weighted=weighted), _same,
                    out=(2,) if weighted else (1,))


def _softmax(B, D, label):
    from .ops.softmax import SoftmaxOp

    return Workload(label, f"X ({B}, {D}) fp32", lambda b: SoftmaxOp(B, D, backend=b), _same, out=(1,))


def _softmax_n():
    from .ops.softmax import SoftmaxOp

    def data(ref_op, device):
        X = workloads.config_n(device, parts=("softmax",))["softmax"]
        return (X, torch.empty_like(X)), (X, torch.empty_like(X))

    return Workload("config-N2-4096x32768", "X (4096, 32768) fp32 ~ N(0, 3)",
                    lambda b: SoftmaxOp(4096, 32768, backend=b), data, out=(1,), repeat=20)


def _reduce(n, label, repeat=2000):
    from .ops.reduce import ReduceOp

    return Workload(label, f"A ({n},) fp32", lambda b: ReduceOp(n, backend=b), _same, out=(1,), repeat=repeat)


def _reduce_n():
    from .ops.reduce import ReduceOp

    def data(ref_op, device):
        A = workloads.config_n(device, parts=("sum",))["sum"]
        o = torch.empty(1, device=device)
        return (A, o), (A, o.clone())

    return Workload("config-N3-2^28", "A (2^28,) fp32 ~ U(-1, 1)", lambda b: ReduceOp(1 << 28, backend=b), data,
                    out=(1,), repeat=20)


# ---- attention (reference: benchmarks/bench_attn_decode.py:28-39) ---------
def _attn(B, H, S, D, Hkv, label, cfg_a=False):
    from .ops.attn_decode import AttnDecodeOp

    def data(ref_op, device):
        d = workloads.config_a(device) if cfg_a else ref_op.gen_data(device=device)
        return d, d

    return Workload(label, f"Q ({B}, {H}, 1, {D})  K/V ({B}, {Hkv}, {S}, {D})",
                    lambda b: AttnDecodeOp(B, H, S, D, backend=b, num_kv_heads=Hkv), data,
                    repeat=20 if cfg_a else N_REPEAT)


def _paged_attn(B, H, Hkv, D, P, M, label):
    from .ops.paged_attn_decode import PagedAttnDecodeOp

    def live_bytes(op, args):  # Q, the table, the lengths and the K/V rows below each length
        Q, _, _, bt, lens = args
        return Q.nbytes + bt.nbytes + lens.nbytes + 2 * Hkv * D * 2 * int(lens.long().sum())

    return Workload(label, f"Q ({B}, {H}, 1, {D})  pool ({B * M}, {Hkv}, {P}, {D})  table ({B}, {M})",
                    lambda b: PagedAttnDecodeOp(B, H, Hkv, D, P, M, backend=b), _same, input_bytes=live_bytes)


# ---- fused ops (reference: benchmarks/bench_fused_{qk_norm_rope,o_proj_ffn}.py)
def _qk_rope_bytes(op, args):
    """Bytes the op must read: q, k, v, both norm weights and one cos and one
    sin row per sequence.  (The reference bench counts every argument,
    including the whole KV cache and RoPE tables the op only indexes, which
    makes its theoretical minimum exceed the time of a whole call.)"""
    q, k, v, qw, kw, cos = args[:6]
    return q.nbytes + k.nbytes + v.nbytes + qw.nbytes + kw.nbytes + 2 * q.shape[0] * cos.shape[1] * cos.element_size()


def _qk_rope(B, S, label, H=16, Hkv=8):
    from .ops.fused_qk_norm_rope import FusedQkNormRopeOp

    return Workload(label, f"batch {B}  heads {H}q/{Hkv}kv x 128  cache ({B}, {Hkv}, {S}, 128)  position {S // 2}",
                    lambda b: FusedQkNormRopeOp(B, H, 128, S, S // 2, backend=b, num_kv_heads=Hkv), _same,
                    mutable=(7, 8), input_bytes=_qk_rope_bytes)


def _qk_rope_f1(B):
    from .ops.fused_qk_norm_rope import FusedQkNormRopeOp

    def make(b):  # the positions are the configuration's first draw
        positions = _F1_POS.setdefault(B, workloads.config_f1_positions(B))
        return FusedQkNormRopeOp(B, 32, 128, 32768, positions, backend=b, num_kv_heads=8)

    def data(ref_op, device):
        d = workloads.config_f1(B, device)[1:]
        return d, d

    return Workload(f"config-F1-b{B}", f"batch {B}  heads 32q/8kv x 128  cache ({B}, 8, 32768, 128)", make, data,
                    mutable=(7, 8), input_bytes=_qk_rope_bytes)


_F1_POS: dict = {}

_OPF_SHAPES = {
    "qwen3-0.6b": dict(hidden_size=1024, intermediate_size=3072, num_heads=16, head_dim=128),
    "qwen3-vl-2b": dict(hidden_size=2048, intermediate_size=6144, num_heads=16, head_dim=128),
    "qwen3-8b": dict(hidden_size=4096, intermediate_size=12288, num_heads=32, head_dim=128),
}


def _oproj_ffn(B, key, label, cfg=False):
    from .ops.fused_o_proj_ffn import FusedOProjFfnOp

    s = _OPF_SHAPES[key]

    def data(ref_op, device):
        d = workloads.config_f2(B, device) if cfg else ref_op.gen_data(device=device)
        return d, d

    return Workload(label, f"batch {B}  hidden {s['hidden_size']}  intermediate {s['intermediate_size']}",
                    lambda b: FusedOProjFfnOp(B, backend=b, **s), data)


# ---- Qwen3 layer (reference: benchmarks/bench_qwen3_dense_decode.py:28-43) -
_VL2B = dict(hidden_size=2048, intermediate_size=6144, num_heads=16, head_dim=128, num_kv_heads=8)


def _layer(B, S, label):
    from .ops.qwen3_dense_decode import Qwen3DenseDecodeOp

    return Workload(label, f"batch {B}  hidden 2048  intermediate 6144  heads 16x128 / 8 kv  cache ({B}, 8, {S}, 128)",
                    lambda b: Qwen3DenseDecodeOp(B, S, backend=b, **_VL2B), _same, mutable=(1, 2))


def _layer_l(B):
    lens = workloads.config_l_lens(B)

    def data(ref_op, device):
        d = workloads.config_l(B, device, backend="ref")[1]
        return d, d

    return Workload(f"config-L-b{B}", f"Qwen3-8B layer, batch {B}, kv_lens ~ U[1024, 16384] over 16384 rows",
                    lambda b: workloads.layer_op(B, backend=b), data, mutable=(1, 2),
                    input_bytes=lambda op, args: workloads.layer_bytes(B, lens), repeat=20)


def registry() -> dict[str, OpBench]:
    """Every benchmarked op with its workloads, in the reference benches' order."""
    return {
        "gemv": OpBench("gemv", "GEMV", [_gemv(4096, 2048, "qwen3-vl-2B-qkv-proj"), _gemv_g()]),
        "rmsnorm": OpBench("rmsnorm", "RMSNorm", [
            _rmsnorm(128, 1024, "128x1K"), _rmsnorm(4096, 4096, "4Kx4K"), _rmsnorm(8192, 8192, "8Kx8K"),
            _rmsnorm(64, 4096, "config-N1-64x4096-bf16", weighted=True, dtype=torch.bfloat16)]),
        "softmax": OpBench("softmax", "Softmax", [
            _softmax(128, 1024, "128x1K"), _softmax(4096, 4096, "4Kx4K"), _softmax(8192, 8192, "8Kx8K"),
            _softmax_n()]),
        "reduce": OpBench("reduce", "Reduce", [
            _reduce(1 << 10, "1K"), _reduce(1 << 20, "1M"), _reduce(1 << 24, "16M", repeat=200), _reduce_n()]),
        "attn_decode": OpBench("attn_decode", "AttnDecode", [
            _attn(1, 16, 1024, 128, 16, "qwen3-0.6b-s1k"), _attn(1, 16, 4096, 128, 16, "qwen3-0.6b-s4k"),
            _attn(1, 16, 8192, 128, 16, "qwen3-0.6b-s8k"), _attn(1, 16, 16384, 128, 16, "qwen3-0.6b-s16k"),
            _attn(1, 16, 16385, 128, 16, "qwen3-0.6b-s16k+1"), _attn(1, 16, 32768, 128, 16, "qwen3-0.6b-s32k"),
            _attn(1, 16, 32768, 128, 8, "qwen3-0.6b-s32k-kv8"), _attn(1, 16, 32768, 128, 4, "qwen3-0.6b-s32k-kv4"),
            _attn(1, 16, 32768, 128, 1, "qwen3-0.6b-s32k-kv1"),
            _attn(32, 32, 8192, 128, 8, "config-A-b32-s8k", cfg_a=True)]),
        "paged_attn_decode": OpBench("paged_attn_decode", "PagedAttnDecode", [
            _paged_attn(1, 32, 8, 128, 64, 256, "qwen3-8b-s16k-p64"),
            _paged_attn(16, 32, 8, 128, 64, 128, "qwen3-8b-b16-s8k-p64")]),
        "fused_qk_norm_rope": OpBench("fused_qk_norm_rope", "FusedQkNormRope", [
            _qk_rope(1, 128, "qwen3-s128"), _qk_rope(1, 1024, "qwen3-s1k"), _qk_rope(1, 4096, "qwen3-s4k"),
            _qk_rope(1, 8192, "qwen3-s8k"), _qk_rope(1, 32768, "qwen3-s32k"), _qk_rope_f1(1), _qk_rope_f1(16)]),
        "fused_o_proj_ffn": OpBench("fused_o_proj_ffn", "FusedOProjFfn", [
            _oproj_ffn(1, "qwen3-0.6b", "qwen3-0.6b-b1"), _oproj_ffn(1, "qwen3-vl-2b", "qwen3-vl-2b-b1"),
            _oproj_ffn(1, "qwen3-8b", "config-F2-b1", cfg=True), _oproj_ffn(16, "qwen3-8b", "config-F2-b16", cfg=True)]),
        "qwen3_dense_decode": OpBench("qwen3_dense_decode", "Qwen3DenseDecode", [
            _layer(1, 1024, "qwen3-vl-2b-s1k"), _layer(1, 4096, "qwen3-vl-2b-s4k"),
            _layer(1, 8192, "qwen3-vl-2b-s8k"), _layer(1, 16384, "qwen3-vl-2b-s16k"),
            _layer_l(1), _layer_l(16)]),
    }


# ---- the harness ------------------------------------------------------------
def _outs(res, args, out):
    if out is not None:
        return [args[i] for i in out]
    return list(res) if isinstance(res, (tuple, list)) else [res]


def _sqnr(refs, outs) -> float:
    noise = sig = 0.0
    for r, o in zip(refs, outs, strict=True):
        r = r.detach().double()
        noise += (r - o.detach().double()).pow(2).sum().item()
        sig += r.pow(2).sum().item()
    if noise == 0.0:
        return math.inf
    return 10.0 * math.log10(sig / noise) if sig > 0 else -math.inf


def _fresh_outputs(args, out):
    args = list(args)
    for i in out or ():
        args[i] = torch.empty_like(args[i])
    return args


def accuracy(op, wl: Workload, kargs, ref_outs) -> dict:
    """Check / SQNR / determinism / read-only of one backend (all untimed)."""
    kargs = _fresh_outputs(kargs, wl.out)
    outs = _outs(op(*kargs), kargs, wl.out)
    outs = [o.clone() for o in outs]
    max_diff = max((o.float() - r.float()).abs().max().item() for o, r in zip(outs, ref_outs, strict=True))
    sq = _sqnr(ref_outs, outs)
    chk = op.check(outs if len(outs) > 1 else outs[0], ref_outs if len(ref_outs) > 1 else ref_outs[0])
    passed = bool(chk) and sq >= SQNR_THRESHOLD_DB
    # determinism: two further calls, outputs byte for byte
    o1 = [o.clone() for o in _outs(op(*kargs), kargs, wl.out)]
    o2 = _outs(op(*kargs), kargs, wl.out)
    det = all(bitwise_equal(a, b) for a, b in zip(o1, o2, strict=True))
    # read-only: every input the op does not own
    watch = [i for i, a in enumerate(kargs)
             if isinstance(a, torch.Tensor) and i not in (wl.out or ()) and i not in wl.mutable]
    before = {i: kargs[i].clone() for i in watch}
    op(*kargs)
    ro = all(bitwise_equal(kargs[i], before[i]) for i in watch)
    return {"max_diff": max_diff, "sqnr_db": sq, "pass": passed, "det": det, "readonly": ro, "args": kargs}


def run_workload(ob: OpBench, wl: Workload, backends, profile, device="cuda", timed=True,
                 n_warmup=WARMUP, n_trials=N_TRIALS, n_repeat=None) -> dict:
    """All backends of one workload; returns {sol, ref_ms, rows}.  A backend
    named "ref" goes through the same checks with the reference's layout
    (a self-check of the harness)."""
    from .ops.utils.bench import bench_kernel

    ref_op = wl.make("ref")
    ref_args, kargs = wl.data(ref_op, device)
    ref_args = _fresh_outputs(ref_args, wl.out)
    ref_outs = [o.clone() for o in _outs(ref_op._ref_forward(*ref_args), ref_args, wl.out)]
    roof = ref_op.get_roofline()
    if wl.input_bytes is not None:
        in_bytes = wl.input_bytes(ref_op, kargs)
    else:
        in_bytes = sum(a.nbytes for i, a in enumerate(ref_args)
                       if isinstance(a, torch.Tensor) and i not in (wl.out or ()))
    sol = hardware.compute_sol(roof, profile, in_bytes) if profile else None
    ref_ms = None
    if timed:
        ref_ms = bench_kernel(ref_op._ref_forward, args=tuple(ref_args), n_warmup=n_warmup,
                              n_repeat=n_repeat or wl.repeat, n_trials=n_trials)
    rows = []
    for backend in backends:
        try:
            op = wl.make(backend)
            acc = accuracy(op, wl, ref_args if backend == "ref" else kargs, ref_outs)
            ms = None
            if timed:
                ms = bench_kernel(op, args=tuple(acc["args"]), n_warmup=n_warmup, n_repeat=n_repeat or wl.repeat,
                                  n_trials=n_trials)
            del acc["args"]
            rows.append(dict(backend=backend, **acc, ms=ms,
                             speedup=(ref_ms / ms) if (ms and ref_ms) else None,
                             sol_score=(sol["theo_min_s"] / (ms * 1e-3)) if (ms and sol) else None))
        except Exception as e:  # a backend that cannot take this workload: report, go on
            rows.append(dict(backend=backend, error=f"{type(e).__name__}: {e}"))
    return {"op": ob.name, "workload": wl.label, "shape": wl.shape, "input_bytes": in_bytes,
            "roofline": {"flops": roof.flops, "bytes": roof.bytes}, "sol": sol, "ref_ms": ref_ms, "rows": rows}


def _fmt(v, f="{:.4f}"):
    return "—" if v is None else f.format(v)


def print_tables(ob: OpBench, res: dict) -> None:
    from tabulate import tabulate

    print(f"\n{'=' * 60}\n  {ob.title} workload: {res['workload']}\n  {res['shape']}")
    print(f"  pass = check AND sqnr >= {SQNR_THRESHOLD_DB:.0f} dB; det = byte-identical over 2 calls; "
          f"input = inputs byte-identical after a call\n{'=' * 60}\n")
    rows = []
    for r in res["rows"]:
        if "error" in r:
            print(f"{r['backend']}: {r['error']}")
            continue
        rows.append([r["backend"], f"{r['max_diff']:.2e}",
                     "inf" if math.isinf(r["sqnr_db"]) else f"{r['sqnr_db']:.1f}",
                     "PASS" if r["pass"] else "FAIL", "OK" if r["det"] else "NONDET",
                     "OK" if r["readonly"] else "MUTATED", _fmt(r["ms"]),
                     _fmt(r["speedup"], "{:.2f}x"), _fmt(r["sol_score"], "{:.3f}")])
    sol = res["sol"]
    rows.append(["ref", "—", "—", "—", "—", "—", _fmt(res["ref_ms"]), "1.00x",
                 _fmt(sol["theo_min_s"] / (res["ref_ms"] * 1e-3) if (sol and res["ref_ms"]) else None, "{:.3f}")])
    print(tabulate(rows, headers=["backend", "max_diff", "sqnr(dB)", "result", "det", "input", "latency(ms)",
                                  "speedup", "sol-score"], tablefmt="github"))
    if sol:
        print()
        print(tabulate([["compute time (tf32 peak)", f"{sol['compute_us']:.3f} µs"],
                        ["mem time (fused)", f"{sol['mem_fused_us']:.3f} µs"],
                        ["mem time (unfused)", f"{sol['mem_unfused_us']:.3f} µs"],
                        ["theoretical min", f"{sol['theo_min_us']:.3f} µs"]],
                       headers=["SOL metric", "value"], tablefmt="github"))


def main(argv=None) -> int:
    reg = registry()
    ap = argparse.ArgumentParser(add_help=False, description="Per-op benchmark (check, SQNR, determinism, "
                                 "read-only, latency, sol-score)")
    ap.add_argument("op", choices=sorted(reg) + ["all"])
    ap.add_argument("-h", action="store_true", dest="list_backends", help="list the op's backends and exit")
    ap.add_argument("-k", "--backends", default=None, help="comma-separated backends (ref is always timed)")
    ap.add_argument("-w", "--workloads", default=None, help="comma-separated workload labels (default: all)")
    ap.add_argument("--json", default=None, help="write every record to this file")
    args = ap.parse_args(argv)

    names = sorted(reg) if args.op == "all" else [args.op]
    if args.list_backends:
        for n in names:
            print(f"{n}: available backends: {', '.join(list_backends(n))}")
        return 0
    profile = hardware.device_profile()
    if profile is None:
        print("no hardware profile for this device: sol-score not computed", file=sys.stderr)
    records = []
    for n in names:
        ob = reg[n]
        avail = list_backends(n)
        sel = avail if args.backends is None else [b.strip() for b in args.backends.split(",") if b.strip()]
        bad = [b for b in sel if b != "ref" and b not in avail]
        if bad:
            print(f"unknown backends for {n}: {', '.join(bad)} (available: {', '.join(avail)})")
            return 2
        sel = [b for b in sel if b != "ref"]
        wanted = None if args.workloads is None else set(args.workloads.split(","))
        for wl in ob.workloads:
            if wanted is not None and wl.label not in wanted:
                continue
            res = run_workload(ob, wl, sel, profile)
            print_tables(ob, res)
            records.append(res)
            torch.cuda.empty_cache()
    if args.json:
        with open(args.json, "w") as f:
            for rec in records:  # JSON has no infinity: a bit-exact SQNR is written as "inf"
                for r in rec["rows"]:
                    if isinstance(r.get("sqnr_db"), float) and math.isinf(r["sqnr_db"]):
                        r["sqnr_db"] = "inf"
            json.dump(records, f, indent=1)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
