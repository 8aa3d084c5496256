"""Region timing in the reference's LWP formats.

The reference's generated code calls a begin and an end hook around every
instrumented region; each appends {id, cycles} to a buffer that
``WriteLWPOutput`` prints as ``{"entries": [{"id": .., "cyc": ..}, ...]}``
(test/utils/dsp/include/prof_utils.cc:37-60), and the compiler writes
``Location <lines> corresponds to ID <id> | Collected ops: <ops>`` lines that
map ids to source (read by test/python/process_lwp.py:63-88).  Here a region
is the GPU work of one planned op: ``LwpRecorder.mark`` enqueues the
``hxmi_lwp_record`` marker on the current stream, so consecutive marks with
one id bracket the kernels launched between them.  ``cyc`` counts ticks of
the GPU's constant-rate wall clock (``cyc_hz`` per second, stored beside the
entries), since GPU shader clocks vary with load.
"""
from __future__ import annotations

import json
from typing import Iterable, Sequence

import torch


class LwpRecorder:
    """Begin/end records on the GPU timeline, in a device buffer of
    ``capacity`` three-word records."""

    def __init__(self, device: torch.device, capacity: int = 8192):
        from .. import hxmi

        self._hxmi = hxmi
        self._lib = hxmi.load_library()
        self.device = device
        self.capacity = int(capacity)
        self.buf = torch.zeros(3 * self.capacity, dtype=torch.int32, device=device)
        self.slot = 0

    def mark(self, region_id: int) -> None:
        """Record `region_id` with the time at which the GPU reaches this point
        of the current stream."""
        if self.slot >= self.capacity:
            raise self._hxmi.HxmiError(f"LWP record buffer full ({self.capacity} records)")
        self._hxmi._check(self._lib.hxmi_lwp_record(self.buf.data_ptr(), self.slot, int(region_id) & 0xFFFFFFFF,
                                                    self._hxmi._stream(self.buf)))
        self.slot += 1

    def entries(self) -> list[dict]:
        """The records so far, in order, as {"id", "cyc"} (waits for the GPU)."""
        torch.cuda.synchronize(self.device)
        words = self.buf[: 3 * self.slot].cpu().numpy().view("uint32").reshape(-1, 3).astype("uint64")
        return [{"id": int(r[0]), "cyc": int(r[1] | (r[2] << 32))} for r in words]

    def clock_hz(self) -> int:
        return int(self._lib.hxmi_lwp_clock_hz())


def lwp_json(entries: Sequence[dict], cyc_hz: int) -> str:
    """The reference's lwp.json layout (prof_utils.cc:37-60), plus the tick
    rate of ``cyc``."""
    lines = ["{", f'  "cyc_hz": {int(cyc_hz)},', '  "entries": [']
    for i, e in enumerate(entries):
        sep = "," if i + 1 < len(entries) else ""
        lines += ["    {", f'      "id": {int(e["id"])},', f'      "cyc": {int(e["cyc"])}', "    }" + sep]
    lines += ["  ]", "}"]
    return "\n".join(lines) + "\n"


def infodump_lines(regions: Iterable[tuple[int, Sequence[int], Sequence[str]]]) -> str:
    """``Location <locs> corresponds to ID <id> | Collected ops: <ops>`` per
    region (id, locations, op names), the id-to-source map process_lwp.py
    reads; a location here is the op's position in the planned graph."""
    out = []
    for rid, locs, ops in regions:
        out.append(f"Location {', '.join(str(int(l)) for l in locs)} corresponds to ID {int(rid)} | "
                   f"Collected ops: {', '.join(ops)}")
    return "\n".join(out) + "\n"


def write_lwp(path_json: str, path_dump: str, entries: Sequence[dict], cyc_hz: int,
              regions: Iterable[tuple[int, Sequence[int], Sequence[str]]]) -> None:
    with open(path_json, "w") as f:
        f.write(lwp_json(entries, cyc_hz))
    with open(path_dump, "w") as f:
        f.write(infodump_lines(regions))


def parse_lwp_json(text: str) -> dict:
    return json.loads(text)
