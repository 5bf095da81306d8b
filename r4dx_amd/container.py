"""Trellis linears from an r4dx weight container: the loader half of `__metadata__.quant.trellis`.

Restates the reference's contract (src/model/trellis_meta.h:10-23, 70-209; docs/trellis-kernel.md:105-117, 148-200;
docs/container-format.md:6-27):

* the container is safetensors-shaped -- an 8-byte little-endian header length, a JSON header, the tensors'
  bytes -- with every tensor stored as U8 and `__metadata__` holding nested JSON (so it is parsed here directly,
  not through a safetensors library, whose metadata is strings only);
* `parse_trellis_metadata` returns None when there is no `quant.trellis` block and refuses (ValueError naming the
  file) any format field this runtime does not implement, a malformed `linears` entry, and a container whose
  reconstruction check did not pass;
* a trellis linear `<base>` is `<base>.trellis.w` (U8 [N K KB / 8]: uint32 ring words in the pair grid, the layout
  the kernels read), `<base>.trellis.suh` (U8 [P K, 2]: fp16, P = 2 for a two-part linear) and `<base>.trellis.svh`
  (U8 [N, 2]: fp16); the rate in the metadata is cross-checked against the byte size.
"""
import json
import struct
from dataclasses import dataclass, field

import numpy as np

TRELLIS_BLOCK = 128            # the Hadamard block: granularity of every trellis K, N and part
MAX_PRESCALE_LOG2 = 16         # the converter's prescale range


@dataclass
class TrellisLinearSpec:
    bits: int
    parts: list = field(default_factory=list)   # output rows per part; empty: one part
    prescale_log2: int = 0

    def n_parts(self):
        return len(self.parts) if self.parts else 1


@dataclass
class TrellisSpec:
    prescale_log2: int
    linears: dict

    def hf_tensors(self):
        return sum(L.n_parts() for L in self.linears.values())


def read_header(path):
    """(header dict, byte offset of the tensor data) of a safetensors-shaped file."""
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(n).decode("utf-8"))
    return header, 8 + n


def tensor_bytes(path, header, data_off, name):
    """The U8 tensor `name` as a read-only numpy memmap of its shape."""
    if name not in header:
        raise KeyError(f"{path}: no tensor {name!r}")
    e = header[name]
    if e.get("dtype") != "U8":
        raise ValueError(f"{path}: tensor {name!r} is {e.get('dtype')}, every r4dx tensor is U8")
    b, en = e["data_offsets"]
    shape = tuple(int(s) for s in e["shape"])
    if en - b != int(np.prod(shape)):
        raise ValueError(f"{path}: tensor {name!r}: data_offsets [{b}, {en}) do not hold shape {shape}")
    return np.memmap(path, dtype=np.uint8, mode="r", offset=data_off + b, shape=shape)


def parse_trellis_metadata(metadata, path):
    """trellis_meta.h:70-209 ParseTrellisMetadata. None without a quant.trellis block."""
    if not isinstance(metadata, dict) or "quant" not in metadata:
        return None
    quant = metadata["quant"]
    if not isinstance(quant, dict) or "trellis" not in quant:
        return None

    def fail(what):
        raise ValueError(f"r4dx_amd.container: {path}: __metadata__.quant.trellis {what} -- refusing to load: its "
                         f"weights would decode to other numbers than the ones converted")

    t = quant["trellis"]
    if not isinstance(t, dict):
        fail("is not an object")

    def str_is(obj, key, want, where=""):
        if not isinstance(obj.get(key), str) or obj[key] != want:
            fail(f'"{where}{key}" is {json.dumps(obj.get(key)) if key in obj else "missing"}, '
                 f'this runtime implements "{want}" only')

    def int_is(obj, key, want, where=""):
        v = obj.get(key)
        if not (isinstance(v, int) and not isinstance(v, bool)) or v != want:
            fail(f'"{where}{key}" is {json.dumps(v) if key in obj else "missing"}, this runtime implements {want} only')

    str_is(t, "format", "r4dx-trellis")
    int_is(t, "version", 1)
    str_is(t, "codebook", "mul1")
    cc = t.get("codebook_consts")
    if not isinstance(cc, dict):
        fail('has no "codebook_consts" object')
    str_is(cc, "mult", "0x83dcd12d", "codebook_consts.")
    str_is(cc, "k_inv_f16", "0x1eee", "codebook_consts.")
    str_is(cc, "k_bias_f16", "0xc931", "codebook_consts.")
    int_is(t, "state_bits", 16)
    if t.get("tail_biting") is not True:
        fail('"tail_biting" is not true')
    str_is(t, "position_order", "exl3-tensor-core")
    str_is(t, "bitstream", "ring-u32-msb-first")
    str_is(t, "tile_grid", "n32-pairs-k-major")
    had = t.get("hadamard")
    if not isinstance(had, dict):
        fail('has no "hadamard" object')
    int_is(had, "block", TRELLIS_BLOCK, "hadamard.")
    str_is(had, "order", "sylvester-natural", "hadamard.")
    str_is(had, "scale", "1/sqrt(128)", "hadamard.")
    str_is(had, "input", "x*suh then H", "hadamard.")
    str_is(had, "output", "H then *svh", "hadamard.")

    def prescale(obj, where):
        s = obj["prescale_log2"]
        if not isinstance(s, int) or isinstance(s, bool):
            fail(f'"{where}" is not an integer')
        if not -MAX_PRESCALE_LOG2 <= s <= MAX_PRESCALE_LOG2:
            fail(f'"{where}" = {s} is outside [-16, 16]')
        return s

    if "prescale_log2" not in t:
        fail('has no "prescale_log2"')
    spec = TrellisSpec(prescale(t, "prescale_log2"), {})
    lin = t.get("linears")
    if not isinstance(lin, dict) or not lin:
        fail('has no non-empty "linears" object')
    for base, e in lin.items():
        where = f"linears.{base}."
        if not base:
            fail('"linears" has an empty base name')
        if not isinstance(e, dict):
            fail(f'"{where[:-1]}" is not an object')
        for k in e:
            if k not in ("bits", "parts", "prescale_log2"):
                fail(f'"{where}{k}" is not a field this runtime knows (bits, parts, prescale_log2)')
        bits = e.get("bits")
        if not isinstance(bits, int) or isinstance(bits, bool):
            fail(f'"{where}bits" is missing or not an integer')
        if bits not in (3, 4, 5):
            fail(f'"{where}bits" = {bits} is not a rate of this format (3, 4, 5)')
        parts = []
        if "parts" in e:
            p = e["parts"]
            if not isinstance(p, list) or len(p) != 2:
                fail(f'"{where}parts" is not an array of two')
            for v in p:
                if not isinstance(v, int) or isinstance(v, bool) or v <= 0 or v % TRELLIS_BLOCK:
                    fail(f'"{where}parts" = {json.dumps(p)} is not two positive multiples of 128')
            parts = list(p)
        ps = prescale(e, where + "prescale_log2") if "prescale_log2" in e else spec.prescale_log2
        spec.linears[base] = TrellisLinearSpec(bits, parts, ps)

    # the converter's own verdict on the bytes it wrote
    def unverified(why):
        raise ValueError(f"r4dx_amd.container: {path} is a trellis container whose reconstruction check did not "
                         f"pass ({why}) -- refusing to load it")

    run = metadata.get("r4dx_convert_run")
    verify = run.get("trellis", {}).get("verify") if isinstance(run, dict) and isinstance(run.get("trellis"), dict) \
        else None
    if not isinstance(verify, dict):
        unverified("no r4dx_convert_run.trellis.verify record")
    result = verify.get("result")
    if not isinstance(result, str):
        unverified("verify.result is missing")
    if not result.startswith("pass"):
        unverified(f'verify.result is "{result}"')
    if "failed" in verify and (not isinstance(verify["failed"], int) or verify["failed"] != 0):
        unverified(f"verify.failed is {json.dumps(verify['failed'])}")
    if "checked" in verify and (not isinstance(verify["checked"], int) or verify["checked"] != spec.hf_tensors()):
        unverified(f"verify.checked is {json.dumps(verify['checked'])}, the linears stand for "
                   f"{spec.hf_tensors()} HF tensors")
    return spec


@dataclass
class TrellisLinear:
    """One trellis linear, as the kernels take it: words (uint32 pair grid), suh (fp32, one array per part),
    svh (fp32 [N]); K, N, KB, parts, prescale_log2."""
    base: str
    words: np.ndarray
    suh: list
    svh: np.ndarray
    K: int
    N: int
    KB: int
    parts: list
    prescale_log2: int


def load_trellis_linear(path, base, spec=None, header=None):
    """The three tensors of `base` (host numpy arrays), shapes and rate checked against the metadata."""
    if header is None:
        header, off = read_header(path)
    else:
        header, off = header
    if spec is None:
        spec = parse_trellis_metadata(header.get("__metadata__", {}), path)
        if spec is None:
            raise ValueError(f"{path}: not a trellis container (no __metadata__.quant.trellis)")
    L = spec.linears.get(base)
    if L is None:
        raise KeyError(f"{path}: {base!r} is not a trellis linear of this container")
    w = tensor_bytes(path, header, off, base + ".trellis.w")
    suh = tensor_bytes(path, header, off, base + ".trellis.suh")
    svh = tensor_bytes(path, header, off, base + ".trellis.svh")
    if w.ndim != 1 or suh.ndim != 2 or suh.shape[1] != 2 or svh.ndim != 2 or svh.shape[1] != 2:
        raise ValueError(f"{path}: {base}: trellis tensors must be w [bytes], suh [P K, 2], svh [N, 2]")
    P = L.n_parts()
    N = svh.shape[0]
    if suh.shape[0] % P:
        raise ValueError(f"{path}: {base}: suh rows {suh.shape[0]} are not {P} parts")
    K = suh.shape[0] // P
    if K % TRELLIS_BLOCK or N % TRELLIS_BLOCK:
        raise ValueError(f"{path}: {base}: K = {K} and N = {N} must be multiples of 128")
    if L.parts and sum(L.parts) != N:
        raise ValueError(f"{path}: {base}: parts {L.parts} do not add up to N = {N}")
    if w.shape[0] * 8 != N * K * L.bits:
        raise ValueError(f"{path}: {base}: {w.shape[0]} word bytes are not N K bits / 8 = {N * K * L.bits // 8} "
                         f"(bits = {L.bits})")
    words = np.frombuffer(np.ascontiguousarray(w).tobytes(), dtype="<u4").copy()
    suh16 = np.ascontiguousarray(suh).view("<f2").reshape(P, K).astype(np.float32)
    svh32 = np.ascontiguousarray(svh).view("<f2").reshape(N).astype(np.float32)
    return TrellisLinear(base, words, [suh16[p].copy() for p in range(P)], svh32, K, N, L.bits, list(L.parts),
                         L.prescale_log2)


COLUMN_PARALLEL, ROW_PARALLEL = "col", "row"


def rank_slice(lin, rank, tp, kind, segments=None):
    """One tensor-parallel rank's share of a trellis linear, as the reference's shard loader cuts it
    (docs/trellis-kernel.md:187-203, the w4a16 rules of tp_shard.cpp:55-101,259-284):
      column-parallel (gate_up, qkv, z, q, k, v): every output segment split into tp equal runs of rows; the
        words of a run are the contiguous pair rows [n0/32, (n0 + cnt)/32) of the pair grid, svh the same rows,
        suh replicated (all parts, full K); the rank's rows are the segments' runs in order. The segments default
        to the linear's parts; a fused one-input linear names its own (qkv: q, k, v), and every part boundary
        must be a segment boundary, so each rank part is the runs of its part's segments;
      row-parallel (down, o, out_proj): K split into tp equal ranges [k0, k0 + kc); per pair row the k-tiles
        [k0/16, (k0 + kc)/16) (N/32 runs of kc/16 * 16 KB words), suh cut to the range, svh replicated. The rank's
        output is the linear's output transform of its partial sum (the transform is linear), so the ranks'
        outputs add up to the full output.
    Every range must be 128-aligned (both Hadamards and the scale vectors work in 128-blocks); one GPU runs a
    rank's share with the same kernels, whatever the rank."""
    if tp < 1 or not 0 <= rank < tp:
        raise ValueError(f"rank {rank} of tp {tp}")
    KT = lin.K // 16
    tile = 16 * lin.KB                                     # words per (pair, k-tile)
    grid = lin.words.reshape(lin.N // 32, KT, tile)
    if kind == COLUMN_PARALLEL:
        part_rows = list(lin.parts) if lin.parts else [lin.N]
        segs = part_rows if segments is None else list(segments)
        bounds = set(np.cumsum(segs).tolist())
        if sum(segs) != lin.N or not set(np.cumsum(part_rows).tolist()) <= bounds:
            raise ValueError(f"{lin.base}: segments {segs} must add up to N = {lin.N} and refine the parts")
        runs, parts, n0, pend, acc = [], [], 0, iter(np.cumsum(part_rows).tolist()), 0
        pe = next(pend)
        for seg in segs:
            cnt = seg // tp
            if seg % tp or cnt % TRELLIS_BLOCK:
                raise ValueError(f"{lin.base}: segment {seg} does not split into {tp} 128-aligned runs")
            runs.append((n0 + rank * cnt, cnt))
            acc += cnt
            n0 += seg
            if n0 == pe:
                parts.append(acc)
                acc = 0
                pe = next(pend, None)
        words = np.concatenate([grid[a // 32:(a + c) // 32].ravel() for a, c in runs])
        svh = np.concatenate([lin.svh[a:a + c] for a, c in runs])
        return TrellisLinear(f"{lin.base}[col {rank}/{tp}]", words, [u.copy() for u in lin.suh], svh, lin.K,
                             sum(parts), lin.KB, parts if len(parts) > 1 else [], lin.prescale_log2)
    if kind == ROW_PARALLEL:
        if len(lin.suh) != 1:
            raise ValueError(f"{lin.base}: a row-parallel linear has one input part")
        kc = lin.K // tp
        if lin.K % tp or kc % TRELLIS_BLOCK:
            raise ValueError(f"{lin.base}: K = {lin.K} does not split into {tp} 128-aligned ranges")
        k0 = rank * kc
        words = np.ascontiguousarray(grid[:, k0 // 16:(k0 + kc) // 16]).ravel()
        return TrellisLinear(f"{lin.base}[row {rank}/{tp}]", words, [lin.suh[0][k0:k0 + kc].copy()],
                             lin.svh.copy(), kc, lin.N, lin.KB, list(lin.parts), lin.prescale_log2)
    raise ValueError(f"kind must be {COLUMN_PARALLEL!r} or {ROW_PARALLEL!r}")


def write_container(path, metadata, tensors):
    """A safetensors-shaped file with U8 tensors (name -> uint8 array) and nested-JSON metadata -- the writer half,
    for tests and tools (docs/container-format.md:6-27)."""
    header = {"__metadata__": metadata}
    off = 0
    blobs = []
    for name, arr in tensors.items():
        a = np.ascontiguousarray(arr, dtype=np.uint8)
        header[name] = {"dtype": "U8", "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        blobs.append(a.tobytes())
        off += a.nbytes
    h = json.dumps(header).encode("utf-8")
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def trellis_tensors(base, words, suh_parts, svh):
    """The three U8 tensors of a trellis linear from words (uint32), suh parts (float) and svh (float)."""
    return {
        base + ".trellis.w": np.asarray(words, "<u4").view(np.uint8),
        base + ".trellis.suh": np.concatenate([np.asarray(s, np.float16) for s in suh_parts]).view(np.uint8).reshape(-1, 2),
        base + ".trellis.svh": np.asarray(svh, np.float16).view(np.uint8).reshape(-1, 2),
    }
