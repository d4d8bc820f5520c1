"""What the reference's engine loader accepts, restated in Python as a test oracle.

parse_aexrt_engine (native/aexrt_d3d12_runtime.cpp:17560-18593) cannot run here (Windows,
D3D12).  reference_accepts() restates its acceptance rules for sections 1-9 and the
inspector's (src/aexrt/engine.py:336-400, src/aexrt/memory_v2.py:611-700) so that engines
written by aexrt_amd.engine can be checked against them without the product's own parser.
Each check cites the line it follows.  Optional sections 10-11 are not restated (the writer
under test does not emit them).
"""
from __future__ import annotations

import struct
import zlib

NO_OFFSET = (1 << 64) - 1
NO_VALUE = (1 << 32) - 1


class Refused(Exception):
    pass


def _need(cond: bool, why: str) -> None:
    if not cond:
        raise Refused(why)


class _R:
    def __init__(self, b: bytes):
        self.b, self.at = b, 0

    def take(self, fmt: str):
        n = struct.calcsize(fmt)
        _need(self.at + n <= len(self.b), "truncated")
        v = struct.unpack_from(fmt, self.b, self.at)
        self.at += n
        return v


# kernel ids that read a packed weight (RT:17811-17843)
_PACKED_CONV = {32, 33, 34, 39, 43, 44, 45, 47, 48, 49, 50, 51, 52, 53}


def _check(data: bytes) -> None:
    # header (RT:17561-17578)
    _need(len(data) >= 64 and data[:8] == b"AEXRTENG", "magic")
    version, hsize, count, flags, fsize, toc_off, toc_size = struct.unpack_from("<IIIIQQQ", data, 8)
    _need(version == 1 and hsize == 64 and 0 < count <= 64 and fsize == len(data), "header")
    _need(toc_size == count * 32 and toc_off <= len(data) and toc_size <= len(data) - toc_off and flags & 1, "toc")
    # TOC (RT:17580-17597)
    secs = {}
    for i in range(count):
        t, _, off, size, crc, res = struct.unpack_from("<IIQQII", data, toc_off + 32 * i)
        _need(res == 0 and t not in secs and off <= len(data) and size <= len(data) - off, "toc entry")
        body = data[off:off + size]
        _need(zlib.crc32(body) & 0xFFFFFFFF == crc, "crc")
        secs[t] = body
    _need(all(t in secs for t in range(1, 10)), "required sections 1-9 (RT:17598-17599)")
    mem_v2 = len(secs[7]) >= 4 and struct.unpack_from("<I", secs[7])[0] == 2
    # manifest (RT:17605-17621)
    r = _R(secs[1])
    m = r.take("<17I")
    inp_el, arena, _, _ = r.take("<QQff")
    r.take("32s")
    _need(m[0] == 1 and m[1] == 1 and m[2] in (1, 2) and m[3] == 2 and m[4] in (1, 2) and m[5] <= 1, "manifest ids")
    _need(m[6] and m[7] and m[8] and m[12] and m[14] and m[15] < m[12] and m[16] < m[12], "manifest counts")
    _need(inp_el != 0 and arena != 0, "manifest input_elements / arena_nbytes (RT:17621)")
    # values (RT:17645-17689)
    r = _R(secs[2])
    n, res = r.take("<II")
    _need(res == 0 and n == m[12], "values header")
    vals = []
    for i in range(n):
        vid, vf, el, *_shape, off, nb = r.take("<IIQ4IQQ")
        _need(vid == i and el != 0, "value id / elements")
        if vf & 4:
            ok = nb in (el * 4, el * 2) if mem_v2 else nb == el * 4
            _need(off != NO_OFFSET and ok and off <= arena and nb <= arena - off, "arena value range")
        elif not mem_v2 and not vf & 8 and not vf & 2:
            raise Refused("value without storage under a V1 plan")
        else:
            _need(off == NO_OFFSET and nb == 0, "non-arena value with a range")
        vals.append(dict(flags=vf, elements=el, off=off, nb=nb))
    # commands (RT:17691-17733)
    r = _R(secs[3])
    n, res = r.take("<II")
    _need(res == 0 and n == m[14], "commands header")
    cmds = []
    for _ in range(n):
        kind, out, ni, npar, pk, prec = r.take("<6I")
        _need(1 <= kind <= 14 and out < len(vals) and ni <= 32 and npar <= 128 and prec in (1, 2), "command")
        if kind in (1, 2):
            _need(pk <= 54 and not 48 <= pk <= 50, "conv kernel id")
        _need(not (kind == 3 and pk > 3) and not (kind > 3 and pk != 0), "kernel id of a non-conv")
        ins = list(r.take(f"<{ni}I")) if ni else []
        _need(all(v < len(vals) for v in ins), "command input")
        params = list(r.take(f"<{npar}I")) if npar else []
        cmds.append(dict(kind=kind, out=out, ins=ins, params=params, pk=pk, prec=prec))
    _need(r.at == len(r.b), "commands trailing bytes")
    # constants (RT:17735-17764)
    r = _R(secs[4])
    n, res = r.take("<II")
    _need(res == 0 and n == m[13], "constants header")
    for _ in range(n):
        vid, dt, el, off, nb = r.take("<IIQQQ")
        _need(vid < len(vals) and dt in (1, 2) and el == vals[vid]["elements"], "constant record")
        _need(nb == el * (2 if dt == 2 else 4) and off <= len(secs[4]) and nb <= len(secs[4]) - off, "constant range")
        _need(vals[vid]["flags"] & 2, "constant of a non-constant value")
    # kernel plan (RT:17766-17887)
    r = _R(secs[5])
    n, pver = r.take("<II")
    _need(n == len(cmds) and pver == 1, "kernel plan header")
    for i in range(n):
        ci, kind, pk, prec, pv, pf = r.take("<6I")
        c = cmds[i]
        _need(ci == i and kind == c["kind"] and prec in (1, 2) and pf & 1 and not pf & ~31, "plan record")
        _need(pk == c["pk"] and prec == c["prec"], "plan vs command")
        conv = kind in (1, 2)
        wants = (conv and (pk in _PACKED_CONV or (pk in (40, 46) and prec == 2 and pf & 2) or (pk == 54 and pf & 2))) \
            or (kind == 3 and pk == 3)
        if wants:
            expect = c["ins"][-2] if kind == 3 else c["ins"][1]
            _need(len(c["ins"]) >= 2 and pv == expect, "plan packed value")
        else:
            _need(pv == NO_VALUE, "packed value on a kernel that reads none")
        native = (kind == 2 and (pk in (43, 44, 47, 48) or (pk in (40, 46) and pf & 2))) or (conv and pk == 45) \
            or (kind == 3 and pk == 3)
        _need(not native or (prec == 2 and pf & 2), "native fp16 kernel plan")
        c["pv"] = pv
    # memory plan (RT:17889-17982; memory_v2.py:611-700)
    r = _R(secs[7])
    if mem_v2:
        _, align, pages, nrec, total, pfl, pres = r.take("<4IQII")
        _need(align >= 4 and align & (align - 1) == 0 and 0 < pages <= 64 and nrec <= len(vals), "memory header")
        _need(total == arena and pfl == 1 and pres == 0, "memory header flags / total")
        pg = []
        for p in range(pages):
            pid, dt, lay, fl, nb = r.take("<4IQ")
            _need(pid == p and dt in (1, 2) and lay in (1, 2) and not (lay == 2 and dt != 2), "page")
            _need(fl == 1 and nb and nb % align == 0 and nb <= total - sum(x[2] for x in pg), "page size")
            pg.append((dt, lay, nb))
        _need(sum(x[2] for x in pg) == total, "page total")
        expect = sum(1 for v in vals if v["off"] != NO_OFFSET and not v["flags"] & 2)
        _need(nrec == expect, "memory record count")
        seen = set()
        for _ in range(nrec):
            vid, vf, page, dt, lay, res, off, nb = r.take("<6IQQ")
            _need(vid < len(vals) and vid not in seen and vf & 4 and page < pages and res == 0, "memory record")
            v = vals[vid]
            _need(dt == pg[page][0] and lay == pg[page][1] and v["off"] == off and v["nb"] == nb, "record vs page")
            _need(nb == v["elements"] * (2 if dt == 2 else 4) and off % align == 0, "record size / alignment")
            _need(off <= pg[page][2] and nb <= pg[page][2] - off, "record inside its page")
            seen.add(vid)
        _need(r.at == len(r.b), "memory plan trailing bytes")
    else:
        align, n, total = r.take("<IIQ")
        _need(align >= 4 and align & (align - 1) == 0 and total == arena, "V1 memory header")
        for _ in range(n):
            vid, vf, off, nb = r.take("<IIQQ")
            _need(vid < len(vals) and vf & 4 and vals[vid]["off"] == off and vals[vid]["nb"] == nb, "V1 record")
        _need(r.at == len(r.b), "V1 memory trailing bytes")
    # packed weights (RT:17984-18040, 18132-18264)
    r = _R(secs[6])
    n, res = r.take("<II")
    _need(res == 0, "packed header")
    packed = {}
    for _ in range(n):
        vid, lay, ic, oc, el, off, nb = r.take("<4IQQQ")
        kk = 16 if lay in (3, 5) else 1 if lay == 4 else (el // (ic * oc) if ic and oc else 0) if lay == 8 \
            else 36 if lay == 9 else 9
        esz = 4 if lay in (1, 5, 7) else 1 if lay == 8 else 2
        _need(vid < len(vals) and 1 <= lay <= 9 and ic and oc, "packed record")
        _need(not (lay == 4 and (ic % 4 or oc % 8)) and not (lay in (6, 7) and (ic % 4 or oc % 4)), "packed shape")
        if lay == 8:
            _need(ic % 4 == 0 and oc % 4 == 0 and el % 4 == 0 and kk in (1, 9) and nb == el + oc * 4, "layout 8")
        _need(el == ic * oc * kk and (lay == 8 or nb == el * esz), "packed elements")
        _need(off <= len(secs[6]) and nb <= len(secs[6]) - off and vid not in packed, "packed range / duplicate")
        _need(vals[vid]["flags"] & 2, "packed weight of a non-constant")
        packed[vid] = (lay, ic, oc, el)
    for c in cmds:
        pv = c["pv"]
        if pv == NO_VALUE:
            continue
        _need(pv in packed, "plan weight not packed")
        lay, ic, oc, el = packed[pv]
        if c["kind"] == 3:
            k = len(c["ins"]) - 2
            _need(lay == 4 and ic == sum(c["params"][5:5 + k]) and oc == c["params"][3], "concat 1x1 weight")
            continue
        p = c["params"]
        _need(len(p) >= 16 and ic == p[1] and oc == p[4], "conv weight channels")
        pk = c["pk"]
        if pk in (51, 52, 53):
            _need(lay == 8 and el == p[1] * p[4] * (1 if pk == 51 else 9), "int8 weight (RT:18132-18164)")
        elif pk == 46:
            _need(lay == 5 and p[:16] == [1, 256, 10, 10, 256, 10, 10, 3, 3, 1, 1, 1, 1, 1, 1, 1], "kernel 46")
        else:
            want = {54: 9, 40: 3, 45: 4, 47: 6, 48: 6, 50: 7}.get(pk)
            _need(lay == want if want else lay in (1, 2), "packed layout of the planned kernel")
            _need(pk not in (43, 44) or lay == 2, "native fp16 weight")
    # fusion plan (RT:18266-18325)
    r = _R(secs[8])
    fver, groups, fcmds, ffl = r.take("<4I")
    _need(fver == 1 and fcmds == len(cmds) and groups <= 2 * fcmds and ffl & 1, "fusion header")
    for _ in range(groups):
        kind, a, b, prec, kern, gf, aux0, aux1 = r.take("<8I")
        _need(1 <= kind <= 9 and a < fcmds and b < fcmds and a <= b and prec in (1, 2) and gf & 1, "fusion group")
    _need(r.at == len(r.b), "fusion trailing bytes")
    # pipeline cache (RT:18556-18590)
    r = _R(secs[9])
    cver, ndxil, npso, _ = r.take("<4I")
    _need(cver == 1 and ndxil + npso <= 4096, "pipeline cache header")
    for _ in range(ndxil + npso):
        kind, rf, key, off, nb = r.take("<IIQQQ")
        _need(kind in (1, 2) and key and nb and not (kind == 1 and rf & ~1) and not (kind == 2 and rf), "cache record")
        _need(off <= len(secs[9]) and nb <= len(secs[9]) - off, "cache payload range")
    # output channels (RT:18592-18593)
    _need(m[8] + (5 if m[5] else 4) <= m[6], "classes vs channels")


def reference_accepts(data: bytes):
    """(True, "") when the reference loader would load the engine, else (False, reason)."""
    try:
        _check(bytes(data))
    except Refused as e:
        return False, str(e)
    return True, ""
