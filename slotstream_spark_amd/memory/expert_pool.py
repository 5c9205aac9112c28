"""Expert slot pool fed from experts.bin, in HBM (drop-in for slotstream_spark/runtime/pool.py's ExpertPool).

The records keep the reference's on-disk format, `slotstream-pool-layer-expert-piece-v1`
(docs/model-and-repack.md:37-57, tools/repack_experts.py:1-9): the record of layer L, expert e at
(L * experts + e) * record_bytes, the nine pieces gate/up/down x weight/scales/biases in that order, described by
experts.manifest.json. The pool itself (slots, CLOCK victims, generation pins, transactional ensure) is native
(`ssmoe_pool_*`); this class owns the two device tables the kernels read, `map` int32 [layers * experts] and
`slot_ptr` int64 [max_slots], and so can stand in for the resident SlotPool in every layer of this package.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import os
from pathlib import Path

import numpy as np
import torch

from .. import _lib

LAYOUT = "slotstream-pool-layer-expert-piece-v1"
PIECE_NAMES = [f"{p}.{k}" for p in ("gate_proj", "up_proj", "down_proj") for k in ("weight", "scales", "biases")]
# record_bytes -> (hidden, moe_intermediate) of the record layouts the kernels know
KNOWN_SHAPES = {2_764_800: (2560, 640), 1_769_472: (2048, 512)}


def read_manifest(packed_dir, manifest_name: str = "experts.manifest.json") -> dict:
    """The manifest with the checks the loader needs: record_bytes / layers / experts present, and, when the full
    manifest is there, its layout name, version, piece names and piece offsets consistent with the record size."""
    man = json.loads((Path(packed_dir) / manifest_name).read_text())
    for k in ("record_bytes", "layers", "experts"):
        if k not in man:
            raise ValueError(f"manifest lacks {k!r}")
    if "layout" in man and man["layout"] != LAYOUT:
        raise ValueError(f"layout {man['layout']!r}, expected {LAYOUT!r}")
    if "version" in man and int(man["version"]) != 1:
        raise ValueError(f"manifest version {man['version']}, expected 1")
    if "piece_names" in man and list(man["piece_names"]) != PIECE_NAMES:
        raise ValueError(f"piece names {man['piece_names']}, expected {PIECE_NAMES}")
    if "piece_offsets" in man:
        offs = [int(x) for x in man["piece_offsets"]]
        if offs[0] != 0 or any(b < a for a, b in zip(offs, offs[1:])) or offs[-1] >= int(man["record_bytes"]):
            raise ValueError(f"piece offsets {offs} do not fit a record of {man['record_bytes']} bytes")
        if "pieces" in man and [int(x) for x in man["pieces"]] != [int(x) for x in np.diff(offs + [man["record_bytes"]])]:
            raise ValueError("piece sizes disagree with piece offsets")
    return man


def write_experts_bin(out_dir, records: np.ndarray, *, model_identity: str = "synthetic",
                      piece_offsets: list[int] | None = None, alignment: int = 4096) -> dict:
    """experts.bin + experts.manifest.json from uint8 records [layers, experts, record_bytes], in the reference's
    format (the fields tests/t0/test_repack_experts.py checks). For synthetic pools and tests; repacking a real
    checkpoint is the reference's tool."""
    rec = np.ascontiguousarray(records, dtype=np.uint8)
    layers, experts, record_bytes = rec.shape
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    data = out / "experts.bin"
    with open(data, "wb") as f:
        for L in range(layers):
            f.write(rec[L].tobytes())
    if piece_offsets is None:
        piece_offsets = [0] * 9
        if record_bytes in KNOWN_SHAPES:
            piece_offsets, _ = _lib.record_layout(*KNOWN_SHAPES[record_bytes])
    st = os.stat(data)
    man = {
        "version": 1, "layout": LAYOUT, "model_identity": model_identity, "layers": layers, "experts": experts,
        "pieces": [int(x) for x in np.diff(list(piece_offsets) + [record_bytes])], "piece_names": PIECE_NAMES,
        "piece_offsets": [int(x) for x in piece_offsets], "record_bytes": record_bytes, "alignment": alignment,
        "layer_sha256": [hashlib.sha256(rec[L].tobytes()).hexdigest() for L in range(layers)],
        "stamp": {"size": st.st_size, "mtime_ns": st.st_mtime_ns}, "total_bytes": layers * experts * record_bytes,
    }
    (out / "experts.manifest.json").write_text(json.dumps(man))
    return man


class PoolView:
    """The `pool` attribute of the reference's ExpertPool (slotio.Pool, pool.hpp:39-92) as far as callers read it:
    slot bytes, the map table, the slot and chunk counts. Slots live in HBM, so slot_view returns a host copy."""

    def __init__(self, owner: "ExpertPool"):
        self._owner = owner

    def slot_view(self, slot, nbytes=None) -> np.ndarray:
        return np.frombuffer(self._owner.slot_bytes(slot, nbytes), dtype=np.uint8)

    def map_numpy(self) -> np.ndarray:
        return self._owner.map_numpy()

    def slot_dev(self, slot) -> int:
        return int(self._owner.slot_ptr[int(slot)].item())

    @property
    def slots(self) -> int:
        return self._owner.stats()["slots"]

    @property
    def chunks(self) -> int:
        return self._owner.stats()["chunks"]

    def owned_bytes(self) -> int:
        return self._owner.owned_bytes()

    def stats(self) -> dict:
        return self._owner.stats()


class ExpertPool:
    """Slots of expert records read from experts.bin with an exact, transactional ensure (runtime/pool.py:27-112).

    `hidden` / `inter` name the record layout for the kernels (inferred from record_bytes for the known shapes).
    `lanes` reader threads (1..12) read the misses of one ensure in parallel; `direct` reads with O_DIRECT (the
    reference's File.open_direct). `mem_type` is accepted for the reference's signature: the slots are always HBM
    here."""

    def __init__(self, packed_dir, slots, mem_type=None, *, experts_name="experts.bin",
                 manifest_name="experts.manifest.json", chunk_bytes=1 << 30, max_slots=25088, hidden=None,
                 inter=None, device="cuda", lanes=4, direct=False):
        packed = Path(packed_dir)
        man = read_manifest(packed, manifest_name)
        self.record_bytes = int(man["record_bytes"])
        layers, experts = int(man["layers"]), int(man["experts"])
        # the MTP layer (index 48) shares the table: 49 layers in the map, 48 in the manifest (runtime/pool.py:37-38)
        self.layers = layers + 1 if layers == 48 else layers
        self.experts = experts
        shape = KNOWN_SHAPES.get(self.record_bytes)
        self.hidden = hidden if hidden is not None else (shape[0] if shape else None)
        self.inter = inter if inter is not None else (shape[1] if shape else None)
        if self.hidden is not None and "piece_offsets" in man:
            offs, nbytes = _lib.record_layout(self.hidden, self.inter)
            if nbytes != self.record_bytes or offs != [int(x) for x in man["piece_offsets"]]:
                raise ValueError(f"manifest piece offsets {man['piece_offsets']} are not the record layout of "
                                 f"hidden {self.hidden}, intermediate {self.inter}")
        self.mem_type = mem_type
        self.device = torch.device(device)
        self.max_slots = int(max_slots)
        self.map = torch.full((self.layers * experts,), -1, dtype=torch.int32, device=self.device)
        self.slot_ptr = torch.zeros(self.max_slots, dtype=torch.int64, device=self.device)
        h = ctypes.c_void_p()
        with torch.cuda.device(self.device):  # the native pool allocates on, and stays bound to, this device
            _lib.check(_lib.lib().ssmoe_pool_open(str(packed / experts_name).encode(), self.layers, experts,
                                                  self.record_bytes, self.max_slots, int(chunk_bytes),
                                                  self.map.data_ptr(), self.slot_ptr.data_ptr(), ctypes.byref(h)))
        self._h = h
        self._gen = 0
        self._progress = None
        self.last_timing = None
        self.pool = PoolView(self)
        self.set_reader(lanes, direct)
        self.resize_slots(slots)

    # The table names of the reference (runtime/pool.py:89-100) and of the resident SlotPool.
    @property
    def map_tensor(self) -> torch.Tensor:
        return self.map

    @property
    def slot_ptr_tensor(self) -> torch.Tensor:
        return self.slot_ptr

    @property
    def n_slots(self) -> int:
        return self.max_slots

    def ensure(self, layer, ids, gen=None) -> np.ndarray:
        """Slot of every id (int32 array, input order). Raises _lib.Exhausted / _lib.IoError, publishing nothing."""
        if gen is None:
            self._gen += 1
            gen = self._gen
        ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
        out = np.empty(ids.size, dtype=np.int32)
        t = np.zeros(6, dtype=np.int64)
        try:
            with torch.cuda.device(self.device):
                _lib.check(_lib.lib().ssmoe_pool_ensure(self._h, int(layer), ids.ctypes.data, ids.size, int(gen),
                                                        out.ctypes.data, t.ctypes.data))
        finally:
            self.last_timing = dict(zip(("hits", "misses", "bytes", "total_ns", "read_ns", "copy_ns"), t.tolist()))
        return out

    def set_reader(self, lanes: int, direct: bool = False) -> None:
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().ssmoe_pool_set_reader(self._h, int(lanes), int(bool(direct))))

    def load_all(self, layers=None, gen=None) -> None:
        """Every expert of the given layers (default: all the file holds) resident, one ensure per layer: the
        pre-fill of a pool with a slot for every record."""
        for layer in range(self.layers if layers is None else layers):
            self.ensure(layer, np.arange(self.experts, dtype=np.int32), gen)

    def resize_slots(self, n) -> None:
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().ssmoe_pool_resize(self._h, int(n)))

    @property
    def slots(self) -> int:
        return self.stats()["slots"]

    def set_progress_ptr(self, addr) -> None:
        """A host progress word (e.g. a pinned int64 a kernel advances): ensure retires the pins below it."""
        _lib.check(_lib.lib().ssmoe_pool_set_progress(self._h, int(addr) if addr else None))

    def retire_below(self, progress) -> None:
        _lib.check(_lib.lib().ssmoe_pool_retire_below(self._h, int(progress)))

    def slot_bytes(self, slot, nbytes=None) -> bytes:
        """The first `nbytes` (default: one record) of a slot, copied to the host (the reference's slot_view)."""
        n = self.record_bytes if nbytes is None else int(nbytes)
        buf = np.empty(n, dtype=np.uint8)
        _lib.check(_lib.lib().ssmoe_pool_copy_slot(self._h, int(slot), buf.ctypes.data, n))
        return buf.tobytes()

    def map_numpy(self) -> np.ndarray:
        return self.map.cpu().numpy()

    def owned_bytes(self) -> int:
        return self.stats()["owned_bytes"]

    def stats(self) -> dict:
        s = np.zeros(10, dtype=np.int64)
        _lib.check(_lib.lib().ssmoe_pool_stats(self._h, s.ctypes.data))
        return dict(zip(("slots", "chunks", "pinned", "owned_bytes", "stride", "hits", "misses", "bytes", "lanes",
                         "direct"), (int(v) for v in s)))

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.lib().ssmoe_pool_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
