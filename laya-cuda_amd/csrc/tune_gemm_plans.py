"""Regenerate gemm_plans.inc: measured (tile, split-K) launches for the batch-1 GEMM problems.

For every encoder shape family below, every packed-row class up to 2,048 rows (the classes
laya_cuda.runtime rounds requests to) and both MFMA input types, each GEMM of the forward is timed
through the op-level C ABI (laya_op_linear / laya_op_qkv) with every tile id and, for the fp32
split-K epilogue, 1/2/4/8 splits, and also with the library's own heuristic plan (tile -2); the
launches take twelve input and weight matrices in turn, so each reads its operands from beyond L2
as a forward does.  A
problem gets a table row only when the best measured launch beats the heuristic by more than 3%;
the library looks rows up at slot creation (exact match on CUs, M, N, K, epilogue, type, RoPE).

Run on the target GPU from the repository root, then rebuild:
    python laya-cuda_amd/csrc/tune_gemm_plans.py [--out path]
"""
import argparse
import ctypes as ct
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "laya-cuda_amd"))

import torch  # noqa: E402

from laya_cuda import _lib  # noqa: E402

# Epilogue ids of the library (kernels.hpp Epi) and op-level linear kinds.
F32, HALF, GELU, QKV, RELU, GEGLU = 0, 1, 2, 3, 4, 5
KIND = {F32: 0, HALF: 1, GELU: 2, RELU: 3, GEGLU: 4}
DTYPE_ID = {"f16": 1, "bf16": 2}  # kernels.hpp DType

LAYERS = 12  # weight matrices timed in turn

# (name, width d, FFN width f, ModernBERT variant)
FAMILIES = [("bert-768", 768, 3072, False), ("bert-1024", 1024, 4096, False), ("modernbert-768", 768, 1152, True)]


def row_classes(limit=2048):
    """Packed-row classes of laya_cuda.runtime._round_rows up to `limit`."""
    out, m = [], 32
    while m <= limit:
        out.append(m)
        m += 32 if m < 256 else 64 if m < 512 else 128
    return out


def problems(d, f, modern):
    """(epilogue, N, K, rope) of each GEMM a forward of this family runs on all rows."""
    if not modern:
        return [(QKV, 3 * d, d, False), (F32, d, d, False), (GELU, f, d, False), (F32, d, f, False)]
    return [(QKV, 3 * d, d, True), (F32, d, d, False), (GEGLU, 2 * f, d, False), (F32, d, f, False),
            (QKV, 3 * d, d, False), (RELU, 4 * d, d, False), (F32, d, 4 * d, False)]


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out", default=str(Path(__file__).with_name("gemm_plans.inc")))
    ap.add_argument("--max-rows", type=int, default=2048)
    args = ap.parse_args()
    lib = _lib.load()
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    stream = ct.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ct.c_void_p(t.data_ptr()) if t is not None else None
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(call):
        """Best of three timings of five back-to-back launches (us per launch); None if refused."""
        if call() != 0:
            return None
        best = None
        for _ in range(3):
            start.record()
            for _ in range(5):
                call()
            end.record()
            end.synchronize()
            us = start.elapsed_time(end) * 1e3 / 5
            best = us if best is None else min(best, us)
        return best

    rows, seen, began = [], set(), time.time()
    maxm = args.max_rows
    for name, d, f, modern in FAMILIES:
        for dtype in ("f16", "bf16"):
            tdt = torch.float16 if dtype == "f16" else torch.bfloat16
            lib_dtype = _lib.F16 if dtype == "f16" else _lib.BF16
            for epi, N, K, rope in problems(d, f, modern):
                # One input and one weight matrix per layer, used in turn: as in a forward, each launch
                # reads operands that are not in its L2 (a loop over one pair would time L2-resident ones).
                xs = [torch.zeros(maxm, K, device=dev, dtype=tdt) for _ in range(LAYERS)]
                ws = [(torch.randn(N, K, device=dev) * 0.02).to(tdt) for _ in range(LAYERS)]
                turn = [0]
                out = torch.zeros(8 * maxm * N, device=dev)  # fp32 partials, or 16-bit outputs
                cos = torch.ones(maxm, 32, device=dev) if rope else None
                sin = torch.zeros(maxm, 32, device=dev) if rope else None
                pos = torch.zeros(maxm, dtype=torch.int32, device=dev) if rope else None
                for M in row_classes(maxm):
                    key = (M, N, K, epi, dtype, rope)
                    if key in seen:  # the same problem in another family: measured once
                        continue
                    seen.add(key)

                    def launch(tile, splits):
                        def call():
                            x, w = xs[turn[0] % LAYERS], ws[turn[0] % LAYERS]
                            turn[0] += 1
                            if epi == QKV:
                                third = M * (N // 3) // 2  # fp32 slots holding M*(N/3) 16-bit values
                                q, k, vt = out[:third], out[third:2 * third], out[2 * third:3 * third]
                                return lib.laya_op_qkv(p(x), p(w), None, p(q), p(k), p(vt), p(cos), p(sin), p(pos),
                                                       lib_dtype, M, N // 3, tile, stream)
                            return lib.laya_op_linear(p(x), p(w), None, p(out), KIND[epi], lib_dtype, M, N, K, splits,
                                                      tile, stream)
                        return call
                    heuristic = timed(launch(-2, 1))
                    best = None
                    for tile in range(64):  # ids past the tile menu are refused (not timed)
                        for splits in ((1, 2, 4, 8) if epi == F32 else (1,)):
                            if splits > 1 and K // 64 // splits < 2:
                                continue
                            us = timed(launch(tile, splits))
                            if us is not None and (best is None or us < best[0]):
                                best = (us, tile, splits)
                    if heuristic is None or best is None:
                        continue
                    gain = 1 - best[0] / heuristic
                    if gain > 0.03:
                        rows.append((cus, M, N, K, epi, DTYPE_ID[dtype], int(rope), best[1], best[2], heuristic, best[0]))
                    print(f"{name} {dtype} epi {epi} M={M} N={N} K={K} rope={int(rope)}: heuristic {heuristic:.2f} us, "
                          f"best t{best[1]} s{best[2]} {best[0]:.2f} us ({gain * 100:+.1f}%)", flush=True)
                del xs, ws, out
                torch.cuda.empty_cache()
    with open(args.out, "w") as fh:
        fh.write("// Measured GEMM plans: {CUs, M, N, K, epilogue, MFMA type, RoPE, tile, splits}.  Each GEMM of the\n"
                 f"// forward at every packed-row class up to {maxm:,} rows was timed on {torch.cuda.get_device_name(0)} "
                 f"({cus} CUs)\n"
                 "// through laya_op_linear / laya_op_qkv with every tile id (and 1/2/4/8 splits for the fp32 split-K\n"
                 "// epilogue) against the heuristic plan (tile -2); a row is kept only where the best measured\n"
                 "// launch beat the heuristic by more than 3% (heuristic -> measured us per launch).  Regenerate on\n"
                 "// the target GPU from the repository root with  python laya-cuda_amd/csrc/tune_gemm_plans.py\n"
                 "// (it rewrites this file), then rebuild the library.\n")
        for cus_, M, N, K, epi, dt, rope, tile, splits, h, b in rows:
            fh.write(f"    {{{cus_}, {M}, {N}, {K}, {epi}, {dt}, {rope}, {tile}, {splits}}},  // {h:.2f} -> {b:.2f}\n")
    print(f"{len(rows)} plans written to {args.out} in {time.time() - began:.0f} s", flush=True)


if __name__ == "__main__":
    main()
