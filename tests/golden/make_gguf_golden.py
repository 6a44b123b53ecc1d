"""Write tests/golden/gguf_cases.json from the COMPILED REFERENCE.

Run where /root/reference exists and `make -C oracle` has built
oracle/_ref/libref.so (the reference's own C sources, compiled unchanged):

    python tests/golden/make_gguf_golden.py

Records, as plain JSON data:
  qwen3_tiny   size and SHA-256 of the GGUF the reference's writer
               (ingot_gguf_writer_save) makes of the tiny Qwen3 at n_ctx 49 —
               the file the qwen3_tiny.npz tokens were decoded from;
  open         for every case of tests/gguf_cases.py OPEN_CASES, what
               ingot_gguf_open reads (null when it refuses the file): version,
               metadata count, alignment, data base, tensor table, and the
               u64 / f64 / string / array-length reads of every key;
  config       for every CONFIG_CASES file, mynah_slm_load's config (null when
               it refuses the file);
  split        for every SPLIT_CASES checkpoint, what ingot_gguf_open_split
               reads (null when it refuses it), each tensor row with its shard.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import json
import os
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "tests"), os.path.join(ROOT, "mynah-slm_amd")]

import configs as CF  # noqa: E402
import gguf_cases as GC  # noqa: E402
import oracle_lib as O  # noqa: E402

TINY_N_CTX = 49          # 16 prefilled positions + 32 steps + 1, as qwen3_tiny.npz


def main() -> None:
    ref = O.load_ref()
    if ref is None:
        sys.exit("oracle/_ref/libref.so is not built (make -C oracle)")
    out = {}
    model = O.SynthModel(CF.QWEN3_TINY, 0)
    err = C.create_string_buffer(512)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tiny.gguf")
        assert ref.ref_write_qwen3_gguf(path.encode(), C.byref(model.c_shape), model.table,
                                        model.count, O.ptr(model.blob), TINY_N_CTX, err,
                                        512) == 0, err.value
        raw = open(path, "rb").read()
        out["qwen3_tiny"] = {"n_ctx": TINY_N_CTX, "bytes": len(raw),
                             "sha256": hashlib.sha256(raw).hexdigest()}
        keys = [k for k, *_ in GC.mini_writer().kvs] + ["general.alignment", "absent.key"]
        out["open"] = {}
        for name, build in GC.OPEN_CASES.items():
            with open(path, "wb") as f:
                f.write(build())
            out["open"][name] = O.ref_gguf_read(ref, path, keys)
        out["config"] = {}
        for name, build in GC.CONFIG_CASES.items():
            with open(path, "wb") as f:
                f.write(build())
            out["config"][name] = O.ref_qwen3_config(ref, path)
        out["split"] = {}
        for name, build in GC.SPLIT_CASES.items():
            files, opened = build()
            sd = os.path.join(d, "split_" + name)
            os.makedirs(sd)
            for fname, data in files:
                with open(os.path.join(sd, fname), "wb") as f:
                    f.write(data)
            out["split"][name] = O.ref_gguf_read(ref, os.path.join(sd, opened), keys, split=True)
    with open(os.path.join(HERE, "gguf_cases.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print("accepted:", sum(v is not None for v in out["open"].values()), "of",
          len(out["open"]), "open cases;", sum(v is not None for v in out["config"].values()),
          "of", len(out["config"]), "config cases;",
          sum(v is not None for v in out["split"].values()), "of", len(out["split"]),
          "split cases")


if __name__ == "__main__":
    main()
