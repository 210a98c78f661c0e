"""QJL hash constants read from the reference's own source text, and the
vectors they define.

The seed mixer `mix_seed` (reference src/qjl.rs:143-147) and the Rademacher
sign hash (src/qjl.rs:157-171) are fixed by integer constants that no
mathematical property pins.  The reference holds them twice: as Rust
`const`s in src/qjl.rs:44-98 and as `#define`s in
src/cache/cuda/kernels/tq_common.h:171-183.  `extract()` reads both copies
as text (nothing of the reference is compiled, imported or run);
`mix_seed()` / `rademacher_sign()` restate the two functions with Python's
exact integers modulo 2^64.

Run as a script (where /root/reference is mounted) to rewrite
tests/golden/qjl_vectors.json: the constants and a grid of
(seed, row) -> mix_seed and (seed, row, col) -> sign, which the tests
compare with the oracle even where the reference is absent.
"""
from __future__ import annotations

import json
import os
import re
import sys

M64 = (1 << 64) - 1
REFERENCE = os.environ.get("TQ_REFERENCE_ROOT", "/root/reference")
RUST_FILE = "src/qjl.rs"
CUDA_FILE = "src/cache/cuda/kernels/tq_common.h"
HERE = os.path.dirname(os.path.abspath(__file__))
VECTORS = os.path.join(HERE, "qjl_vectors.json")

# constant name in qjl.rs -> its #define in tq_common.h (None: only in Rust,
# the CUDA copy writes the shift as a literal in tq_rademacher_sign)
NAMES = {
    "SEED_MIX_MULTIPLIER": "TQ_SEED_MIX_MULTIPLIER",
    "SEED_MIX_XOR": "TQ_SEED_MIX_XOR",
    "SEED_MIX_SHIFT": "TQ_SEED_MIX_SHIFT",
    "SPLITMIX_GAMMA": "TQ_SPLITMIX_GAMMA",
    "SPLITMIX_MUL_1": "TQ_SPLITMIX_MUL_1",
    "SPLITMIX_MUL_2": "TQ_SPLITMIX_MUL_2",
    "SPLITMIX_SHIFT_1": None,
    "SPLITMIX_SHIFT_2": None,
    "SPLITMIX_SHIFT_3": None,
}


def _int(text: str) -> int:
    t = text.replace("_", "").rstrip("ULul")
    return int(t, 16) if t.lower().startswith("0x") else int(t)


def extract(root: str = REFERENCE) -> dict:
    """{"rust": {name: value}, "cuda": {name: value}} from the two source copies."""
    with open(os.path.join(root, RUST_FILE)) as f:
        rust_src = f.read()
    with open(os.path.join(root, CUDA_FILE)) as f:
        cuda_src = f.read()
    rust, cuda = {}, {}
    for name, cname in NAMES.items():
        m = re.search(rf"const\s+{name}\s*:\s*u(?:64|32)\s*=\s*([0-9A-Fa-fxX_]+)\s*;", rust_src)
        if not m:
            raise ValueError(f"{name} not found in {RUST_FILE}")
        rust[name] = _int(m.group(1))
        if cname:
            m = re.search(rf"#define\s+{cname}\s+([0-9A-Fa-fxXuUlL]+)", cuda_src)
            if not m:
                raise ValueError(f"{cname} not found in {CUDA_FILE}")
            cuda[name] = _int(m.group(1))
    # the CUDA copy's finalizer shifts are literals: z ^ (z >> 30), >> 27, >> 31
    shifts = [int(s) for s in re.findall(r"z\s*=\s*\(?z\s*\^\s*\(z\s*>>\s*(\d+)\)", cuda_src)]
    if len(shifts) != 3:
        raise ValueError(f"finalizer shifts not found in {CUDA_FILE}")
    cuda["SPLITMIX_SHIFT_1"], cuda["SPLITMIX_SHIFT_2"], cuda["SPLITMIX_SHIFT_3"] = shifts
    return {"rust": rust, "cuda": cuda}


def mix_seed(k: dict, seed: int, row: int) -> int:
    """qjl.rs:143-147: m = seed * MULT + row (mod 2^64); m ^ (m >> SHIFT) ^ XOR."""
    m = (seed * k["SEED_MIX_MULTIPLIER"] + row) & M64
    return (m ^ (m >> k["SEED_MIX_SHIFT"]) ^ k["SEED_MIX_XOR"]) & M64


def rademacher_sign(k: dict, row_seed: int, row: int, col: int) -> float:
    """qjl.rs:157-171: SplitMix64 finalizer of row_seed + row * gamma + col; +1 if even."""
    z = (row_seed + row * k["SPLITMIX_GAMMA"] + col) & M64
    z = ((z ^ (z >> k["SPLITMIX_SHIFT_1"])) * k["SPLITMIX_MUL_1"]) & M64
    z = ((z ^ (z >> k["SPLITMIX_SHIFT_2"])) * k["SPLITMIX_MUL_2"]) & M64
    z ^= z >> k["SPLITMIX_SHIFT_3"]
    return 1.0 if z % 2 == 0 else -1.0


SEEDS = [0, 1, 42, 777, 4242, 12345, 99999, 0x123456789ABCDEF0, (1 << 63) + 5, M64]
ROWS = [0, 1, 2, 31, 63, 64, 127, 255, 1000, 65535]
COLS = [0, 1, 17, 63, 127]


def vectors(k: dict) -> dict:
    mix = [[hex(s), r, hex(mix_seed(k, s, r))] for s in SEEDS for r in ROWS]
    signs = [[hex(s), r, c, rademacher_sign(k, mix_seed(k, s, r), r, c)] for s in SEEDS[:6] for r in ROWS[:6]
             for c in COLS]
    return {"about": "QJL hash constants of the reference's two source copies and the mix_seed / Rademacher "
                     "sign vectors they define (tests/golden/qjl_reference_constants.py)",
            "source": [RUST_FILE, CUDA_FILE],
            "constants": {n: hex(v) for n, v in k.items()}, "mix_seed": mix, "signs": signs}


def main() -> int:
    both = extract()
    if both["rust"] != both["cuda"]:
        print("the reference's two copies disagree:", both, file=sys.stderr)
        return 1
    with open(VECTORS, "w") as f:
        json.dump(vectors(both["rust"]), f, separators=(",", ":"))
        f.write("\n")
    print(f"wrote {VECTORS}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
