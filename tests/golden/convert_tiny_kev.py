"""Copy the reference's tiny Kev fixture into tests/golden/tiny_kev as data.

Source: crates/huncho-backend/tests/fixtures/tiny_kev in grafuls/huncho (Apache-2.0).
The safetensors/JSON files are copied verbatim. `head.pt` is a PyTorch zip archive; it
is read without unpickling: the four float32 storages are taken from the zip members
`head/data/0..3` and the scalar metadata from the opcode stream of `head/data.pkl`
(pickletools.genops only lists opcodes, it executes nothing). The storage order and
shapes are q.weight [head_dim, hidden], q.bias [head_dim], k.weight, k.bias, as the
opcode listing shows. Run once in the container that has the reference checkout.
"""
import json
import pickletools
import shutil
import sys
import zipfile
from pathlib import Path

import numpy as np

SRC = Path(sys.argv[1] if len(sys.argv) > 1 else
           "/root/reference/crates/huncho-backend/tests/fixtures/tiny_kev")
DST = Path(__file__).resolve().parent / "tiny_kev"


def head_metadata(pkl: bytes) -> dict:
    """Top-level scalar entries of the metadata dict, read from the opcode stream.

    At nesting depth 1 (inside the top-level dict's MARK) a string opcode is either a
    key or a scalar value; any other value-starting opcode (a nested MARK, dict, memo
    lookup or global) means the pending key has a non-scalar value and is dropped."""
    meta, pending, depth = {}, None, 0
    for op, arg, _ in pickletools.genops(pkl):
        name = op.name
        if name == "MARK":
            if depth == 1:
                pending = None
            depth += 1
            continue
        if name in ("TUPLE", "SETITEMS", "LIST", "DICT"):
            depth -= 1
            continue
        if depth != 1:
            continue
        if name == "BINUNICODE":
            if pending is None:
                pending = arg
            else:
                meta[pending], pending = arg, None
        elif name in ("BINFLOAT", "BININT1", "BININT", "BININT2") and pending is not None:
            meta[pending], pending = arg, None
        elif name in ("NEWFALSE", "NEWTRUE") and pending is not None:
            meta[pending], pending = name == "NEWTRUE", None
        elif name in ("EMPTY_DICT", "EMPTY_TUPLE", "EMPTY_LIST", "BINGET", "GLOBAL"):
            pending = None
    return meta


def main() -> None:
    DST.mkdir(parents=True, exist_ok=True)
    for name in ["config.json", "model.safetensors", "adapter_model.safetensors",
                 "adapter_config.json", "golden.json", "README.md"]:
        shutil.copyfile(SRC / name, DST / name)
    z = zipfile.ZipFile(SRC / "head.pt")
    meta = head_metadata(z.read("head/data.pkl"))
    hd = int(meta["head_dim"])
    store = [np.frombuffer(z.read(f"head/data/{i}"), dtype="<f4") for i in range(4)]
    hidden = store[0].size // hd
    head = {
        "head_dim": hd,
        "hidden_size": hidden,
        "temperature": float(meta["temperature"]),
        "lora": int(meta["lora"]),
        "base": meta["base"],
        "weights_dtype": meta["weights_dtype"],
        "q_weight": store[0].reshape(hd, hidden).tolist(),
        "q_bias": store[1].tolist(),
        "k_weight": store[2].reshape(hd, hidden).tolist(),
        "k_bias": store[3].tolist(),
    }
    (DST / "head.json").write_text(json.dumps(head, indent=1))
    print("wrote", DST, {k: v for k, v in head.items() if not isinstance(v, list)})


if __name__ == "__main__":
    main()
