"""The gfx950 GEMM route: which of libhkx.so's kernels an M x N x K call runs.

The reference's `gemm_cdna.route` (python/hk/ops/gemm_cdna.py:969-999) answers from a
measured table (the nearest M on a log scale for that N x K), else a rule (decode for
M <= 32, small blocks to M 2048, the 256 x 256 pingpong above). This is the same
contract over this build's kernels:

* `CANDIDATES` -- the schedules a route may name: the ring and ping-pong kernels at 256 x 256, the
  4-wave 32x32-MFMA tile kernel at 256 / 128 / 64 rows, the 8-wave 16x16-MFMA one, their
  split-K forms, the decode kernel;
* `route(m, n, k)` -- a user record (`OVERRIDE`), else the measured table
  `hk/tuned/routes_gemm_gfx950.json` (this build's own measurements), else `rule`;
* `resolve` -- a candidate made concrete for a shape (the decode kernel's split);
* `fits` -- whether a candidate takes a shape;
* `matmul` -- the plain bf16 GEMM through it (hk.ops.matmul's gfx950 form).
"""

from __future__ import annotations

import json
import math
import os
from pathlib import Path
from typing import Any, Dict, Optional

#: Multiples the kernels need: K in 128-byte stages (64 bf16), N in 4s.
K_STEP = 64
BLOCK_N_MIN = 4
#: A and B are read through buffer resources with 32-bit byte offsets: each spans less
#: than 4 GiB (hkx_gemm refuses larger ones).
OPERAND_BYTES_MAX = 1 << 32
#: CUs of an MI355X.
CUS = 256

CANDIDATES: Dict[str, Dict[str, Any]] = {
    # 256 x 256: the ring kernel (8 waves taking turns at the MFMA, one workgroup a CU
    # walking its tiles through one LDS ring, the epilogue stored from registers), and the
    # ping-pong kernel it is measured against (one tile a workgroup; "t256ppc": one
    # workgroup a CU; "t256m32": 32 x 32 MFMA fragments)
    "t256": {"kernel": "tile", "tile_m": 256, "tile_n": 256, "schedule": "ring"},
    "t256pp": {"kernel": "tile", "tile_m": 256, "tile_n": 256, "schedule": "pp", "variant": 2},
    "t256ppc": {"kernel": "tile", "tile_m": 256, "tile_n": 256, "schedule": "pp"},
    "t256m32": {"kernel": "tile", "tile_m": 256, "tile_n": 256, "schedule": "pp", "variant": 3},
    "t256w4": {"kernel": "tile", "tile_m": 256, "tile_n": 256, "schedule": "w4"},
    "t256w8": {"kernel": "tile", "tile_m": 256, "tile_n": 256, "schedule": "w8"},
    # smaller tiles: the 4-wave kernel (32 x 32 MFMAs), the 8-wave one (16 x 16)
    "t128": {"kernel": "tile", "tile_m": 128, "tile_n": 256, "schedule": "w4"},
    "t64": {"kernel": "tile", "tile_m": 64, "tile_n": 256, "schedule": "w4"},
    "t128w8": {"kernel": "tile", "tile_m": 128, "tile_n": 256, "schedule": "w8"},
    "t64w8": {"kernel": "tile", "tile_m": 64, "tile_n": 256, "schedule": "w8"},
    "t128n128": {"kernel": "tile", "tile_m": 128, "tile_n": 128, "schedule": "w8"},
    "t256n128": {"kernel": "tile", "tile_m": 256, "tile_n": 128, "schedule": "w8"},
    # split over K
    "t256k2": {"kernel": "tile", "tile_m": 256, "tile_n": 256, "schedule": "ring", "splits": 2},
    "t256k4": {"kernel": "tile", "tile_m": 256, "tile_n": 256, "schedule": "ring", "splits": 4},
    "t256k8": {"kernel": "tile", "tile_m": 256, "tile_n": 256, "schedule": "ring", "splits": 8},
    # wave split: the columns whose 256 x 256 tiles fill whole waves of the CUs on the ring
    # kernel, the rest of N on 128 x 256 tiles (gemm_cdna.py:834-835's ppw)
    "t256w": {"kernel": "tile", "tile_m": 256, "tile_n": 256, "schedule": "ring", "variant": 4},
    # stream-K: the whole waves likewise, the rest of N on 256 x 256 tiles split over K to
    # fill the CUs (gemm_cdna.py:421-496's dp+sk mode; the shares summed by one pass)
    "t256sk": {"kernel": "tile", "tile_m": 256, "tile_n": 256, "schedule": "ring", "variant": 8},
    "t128k2": {"kernel": "tile", "tile_m": 128, "tile_n": 256, "schedule": "w4", "splits": 2},
    "t128k4": {"kernel": "tile", "tile_m": 128, "tile_n": 256, "schedule": "w4", "splits": 4},
    "t64k2": {"kernel": "tile", "tile_m": 64, "tile_n": 256, "schedule": "w4", "splits": 2},
    "t64k4": {"kernel": "tile", "tile_m": 64, "tile_n": 256, "schedule": "w4", "splits": 4},
    "t64k8": {"kernel": "tile", "tile_m": 64, "tile_n": 256, "schedule": "w4", "splits": 8},
    # 128 x 256 tiles on the quadrant kernel (8 waves in two ping-pong groups, one phase a
    # K-tile, three LDS slots); calls it does not take run on the 4-wave kernel
    "q128": {"kernel": "tile", "tile_m": 128, "tile_n": 256, "schedule": "ring"},
    # 128-column tiles on the 4-wave kernel (four LDS stages): twice the tiles of the
    # 256-column ones at mid M, so fewer splits fill the CUs (gemm_cdna_dp.py's dp64 / dp128
    # blocks are 128 columns wide)
    "t128x128": {"kernel": "tile", "tile_m": 128, "tile_n": 128, "schedule": "w4"},
    "t128x128k2": {"kernel": "tile", "tile_m": 128, "tile_n": 128, "schedule": "w4", "splits": 2},
    "t128x128k4": {"kernel": "tile", "tile_m": 128, "tile_n": 128, "schedule": "w4", "splits": 4},
    "t64x128": {"kernel": "tile", "tile_m": 64, "tile_n": 128, "schedule": "w4"},
    "t64x128k2": {"kernel": "tile", "tile_m": 64, "tile_n": 128, "schedule": "w4", "splits": 2},
    "t64x128k4": {"kernel": "tile", "tile_m": 64, "tile_n": 128, "schedule": "w4", "splits": 4},
    "t64x128k8": {"kernel": "tile", "tile_m": 64, "tile_n": 128, "schedule": "w4", "splits": 8},
    "decode": {"kernel": "decode", "waves": 8, "rows": 16, "splits": "auto", "variant": 1},
    "decode_blk": {"kernel": "decode", "waves": 8, "rows": 16, "splits": "auto"},
    "decode_w4": {"kernel": "decode", "waves": 4, "rows": 16, "splits": "auto"},
    "decode_w16": {"kernel": "decode", "waves": 16, "rows": 16, "splits": "auto"},
}

#: A user's choice laid over everything: {(m, n, k): candidate} or {"*": candidate}.
OVERRIDE: Dict[Any, str] = {}

TABLE_PATH = Path(__file__).resolve().parents[1] / "tuned" / "routes_gemm_gfx950.json"
_TABLE: list = []


def table() -> Dict[str, Dict[str, str]]:
    """The measured table's routes: {"NxK": {"M": candidate}} ($HK_GEMM_ROUTES names
    another file; `hk.integration.tune gemm` writes one). A table of another arch, or
    naming a candidate this build does not have, is refused."""
    if not _TABLE:
        path = Path(os.environ.get("HK_GEMM_ROUTES", TABLE_PATH))
        routes = {}
        if path.is_file():
            d = json.loads(path.read_text())
            if d.get("arch", "gfx950") != "gfx950":
                raise ValueError(f"{path} was measured on {d['arch']}, not gfx950")
            routes = d.get("routes", {})
            bad = {c for ent in routes.values() for c in ent.values()} - set(CANDIDATES)
            if bad:
                raise ValueError(f"{path} names candidates this build lacks: {sorted(bad)}")
        _TABLE.append(routes)
    return _TABLE[0]


def reload_table() -> None:
    """Read the table again on the next route (after $HK_GEMM_ROUTES changes)."""
    _TABLE.clear()


def fits(name: str, m: int, n: int, k: int, fp8: bool = False) -> bool:
    """Whether candidate `name` takes an M x N x K call."""
    c = CANDIDATES.get(name)
    if c is None or m < 1 or n % BLOCK_N_MIN:
        return False
    kstep = 128 if fp8 else 64
    if k % kstep or max(m, n) * k * (1 if fp8 else 2) >= OPERAND_BYTES_MAX:
        return False
    if c["kernel"] == "decode":
        return not fp8 and m <= 32 and k % 128 == 0
    return True


def rule(m: int, n: int, k: int, fp8: bool = False) -> str:
    """The route when no record or table entry names one: the decode kernel at M <= 32
    (bf16); else the largest tile whose count fills three quarters of the CUs -- 256 x 256,
    128 x 256 (the quadrant kernel's 128-row form for bf16 up to K = 4096, the 4-wave
    kernel otherwise), 128 x 128; else 64 x 128 tiles (up to M = 128) or 128 x 128 ones,
    split over K in powers of two while the workgroups stay within the CUs and each split
    keeps 16 or more 128-byte K units. On the shipped table's 132 measured points its pick
    is 2% slower than the best candidate on average (the rule before the 128-column tiles:
    26%).

    fp8 has no measured table, so its last step follows one measured sweep (scaled_mm with
    dequant and bias, N x K in {4096 x 4096, 12288 x 4096, 4096 x 12288}, M 256-4096, every
    tile candidate, M 16-4096): from M = 129 to 512, 64 x 128 tiles, split only where each
    split keeps 32 K units (4096 x 4096 at M = 256: 12.1-12.2 us on 64 x 128 tiles against
    19.6 on 128 x 128 ones split in two; at M = 512 13.9 against 21.9; 4096 x 12288 at M =
    256 split in two, 23.9 against 29.9 unsplit); up to M = 128 the bf16 steps."""
    if not fp8 and m <= 32 and k % 128 == 0:
        return "decode"
    kunits = k * (1 if fp8 else 2) // 128

    def tiles(bm, bn):
        return math.ceil(m / bm) * math.ceil(n / bn)

    if m > 128 and tiles(256, 256) >= 0.75 * CUS:
        return "t256"
    if m > 64 and tiles(128, 256) >= 0.75 * CUS:
        return "q128" if not fp8 and kunits <= 64 else "t128"
    if m > 64 and tiles(128, 128) >= 0.75 * CUS:
        return "t128x128"
    bm = 64 if m <= (512 if fp8 else 128) else 128
    t = tiles(bm, 128)
    most = 8 if bm == 64 else 4  # the split candidates there are
    per_split = 32 if fp8 and m > 128 else 16  # K units a split keeps at least
    splits = 1
    while t * splits * 2 <= CUS and kunits // (splits * 2) >= per_split and splits < most:
        splits *= 2
    return f"t{bm}x128" + (f"k{splits}" if splits > 1 else "")


def route(m: int, n: int, k: int, fp8: bool = False) -> str:
    """The candidate an M x N x K call runs: a user record, else the measured table's
    nearest M (log scale) for this N x K, else `rule` (gemm_cdna.py:969-999)."""
    for key in ((m, n, k), "*"):
        if key in OVERRIDE and fits(OVERRIDE[key], m, n, k, fp8):
            return OVERRIDE[key]
    if not fp8:
        ent = table().get(f"{n}x{k}")
        if ent:
            ms = sorted(int(x) for x in ent)
            best = min(ms, key=lambda x: abs(math.log(x) - math.log(m)))
            name = ent[str(best)]
            if fits(name, m, n, k, fp8):
                return name
    return rule(m, n, k, fp8)


def resolve(rec: Dict[str, Any], m: int, n: int, k: int, fp8: bool = False) -> Dict[str, Any]:
    """A candidate made concrete for a shape: the decode kernel's split over K (enough
    workgroups for twice the CUs, at least four 128-element groups a split)."""
    rec = dict(rec)
    if rec["kernel"] == "decode" and rec.get("variant", 0) & 1 and k % 1024 == 0 and k <= 32768 \
            and (m <= 16 or (m <= 32 and k >= 2048)) and rec.get("splits") == "auto":
        # the streaming kernel: one workgroup a CU walks all of W, no split (two 16-token
        # fragments from M = 17, with K of 2048 and up)
        rec["splits"] = 1
    if rec["kernel"] == "decode" and rec.get("splits") == "auto":
        wgs = math.ceil(n / (16 * (rec.get("rows", 16) // 16)))
        groups = k // 128
        splits = 1
        while wgs * splits < 2 * CUS and groups // (splits * 2) >= 4:
            splits *= 2
        rec["splits"] = splits
    rec.setdefault("splits", 1)
    return rec


def matmul(a, b, out=None):
    """C = A @ B^T in bf16 (hk.ops.matmul's gfx950 form, gemm_cdna.py:1090): the
    template with no epilogue."""
    from ..templates import gemm as T  # noqa: PLC0415

    return T.gemm(a, b, out=out)


__all__ = ["CANDIDATES", "OVERRIDE", "route", "rule", "resolve", "fits", "matmul", "table",
           "reload_table",
           "K_STEP", "BLOCK_N_MIN", "OPERAND_BYTES_MAX", "CUS"]
