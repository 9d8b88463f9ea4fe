"""Write tests/golden/ref_vectors.npz from the reference's own CPU path (run in the build container only).

The reference extension is compiled from /root/reference/engine/csrc/cpu/qwen_cpu.c into oracle/_ref/ by
`make -C oracle ref`; this script loads that build (never the reference's Python package) and records,
for every quantized type plus F32/F16:
  w_<T>      seeded synthetic blocks (synthetic_rows, the reference tests' recipe), 4 rows
  x_<T>      fp32 activations, 3 tokens
  y_<T>      the reference's Cpu_qmv output (qwen_cpu.c:581-641) for those inputs
  probe_<T>  the reference's output for one-hot activations x = I (ntok = cols): y[c][r] ~ W[r][c]
             (a pin on the decoded value of every element, up to a few ulp of rounding)
sha256_<table>: SHA-256 of every codebook as the reference holds it (iq_tables.py hex, dequant.py:373-414);
and q8_<n>: reference quantize_q8_0 blocks (its own copy of the activation quantizer rule) for a few
activation vectors, pinning the int8 quantizer bit for bit.
"""
from __future__ import annotations

import glob
import importlib.util
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from vinf_3080ti_amd import GGUFTensorType as T  # noqa: E402
from vinf_3080ti_amd import QUANT_TYPES, synth, tables  # noqa: E402

SEED = 20261201


def load_ref():
    paths = glob.glob(str(ROOT / "oracle" / "_ref" / "_cpu_qwen*.so"))
    if not paths:
        raise SystemExit("oracle/_ref is not built: run `make -C oracle ref`")
    spec = importlib.util.spec_from_file_location("_cpu_qwen", paths[0])
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def ref_qmv(rt, name, w, ty, rows, cols, x):
    ntok = x.shape[0]
    rt.add_tensor(name, w.tobytes(), int(ty), cols, rows)
    rt.alloc(name + ".x", cols * ntok)
    rt.alloc(name + ".y", rows * ntok)
    rt.write(name + ".x", np.ascontiguousarray(x, np.float32).tobytes())
    rt.qmv(name, name + ".x", name + ".y", ntok)
    return np.frombuffer(rt.read(name + ".y"), np.float32).reshape(ntok, rows).copy()


def main() -> None:
    ref = load_ref()
    rt = ref.CpuRuntime(tables.table("iq3s_grid"), 1)
    rng = np.random.default_rng(SEED)
    out = {}
    for ty in list(QUANT_TYPES) + [T.F32, T.F16]:
        rows, cols = 4, 512
        w = synth.synthetic_rows(ty, rows, cols, rng)
        x = rng.uniform(-1, 1, (3, cols)).astype(np.float32)
        out[f"w_{ty.name}"] = w
        out[f"x_{ty.name}"] = x
        out[f"y_{ty.name}"] = ref_qmv(rt, f"g{int(ty)}", w, ty, rows, cols, x)
        if ty in QUANT_TYPES:
            pcols = 256
            wp = synth.synthetic_rows(ty, 2, pcols, rng)
            out[f"pw_{ty.name}"] = wp
            out[f"probe_{ty.name}"] = ref_qmv(rt, f"p{int(ty)}", wp, ty, 2, pcols, np.eye(pcols, dtype=np.float32))
    for n in range(4):
        x = (rng.standard_normal(256) * (10.0 ** (n - 2))).astype(np.float32)
        if n == 3:
            x[:32] = 0.0  # an all-zero group (d = 0, id = 0)
            x[40] = 0.5 * x[41]  # keep ordinary values around exact halves
        out[f"q8x_{n}"] = x
        out[f"q8_{n}"] = np.frombuffer(ref.quantize_q8_0(x.tobytes(), 0), np.uint8).copy()
    sys.path.insert(0, str(ROOT / "vinf_3080ti_amd" / "csrc"))
    from gen_iq_grids import reference_tables

    import hashlib

    for name, data in sorted(reference_tables(Path("/root/reference")).items()):
        out[f"sha256_{name}"] = np.frombuffer(hashlib.sha256(data).digest(), np.uint8).copy()
    np.savez_compressed(Path(__file__).with_name("ref_vectors.npz"), **out)
    print("wrote", len(out), "arrays")


if __name__ == "__main__":
    main()
