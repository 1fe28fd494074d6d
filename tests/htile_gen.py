"""HTile flash-attention tile programs for the front-end tests.

``program(...)`` writes the attention tile program in HTile IR for a given
shape and dtype, in the two forms the reference produces: as written
(K tile row-major, ``htile.dot {transpose_b}``) and after its
htile-dot-transpose-to-load-order pass (K tile loaded with
``dimension_order = array<i64: 1, 0>``, no transpose on the dot). With
``canonical=True`` values carry numbered names (``%0``, ``%c0``, ``%cst``,
loop results as ``%r:3`` used as ``%r#i``), ops appear in another order
and a size-1 grid dimension's block id is folded to ``%c0``, as after
canonicalisation. ``k_mem="ds"`` declares K as [B, H, D, S] and loads its
[D, block_n] tile in stored order (no transpose anywhere). ``mutate`` swaps
in one wrong piece for negative tests.
"""

from __future__ import annotations

import math

ELT = {"f16": "f16", "bf16": "bf16", "f32": "f32"}


def program(B=1, H=32, S=4096, D=128, dtype="f16", bm=128, bn=64, form="pre", grid=None,
            threads=128, trip=None, scale=None, stages=2, canonical=False, name="flash_attention_htile",
            mutate=None, k_mem="sd"):
    e = ELT[dtype]
    grid = grid or (S // bm, H, B)
    trip = trip if trip is not None else S // bn
    scale = scale if scale is not None else math.log2(math.e) / math.sqrt(D)
    mem = f"memref<{B}x{H}x{S}x{D}x{e}>"
    kmem = f"memref<{B}x{H}x{D}x{S}x{e}>" if k_mem == "ds" else mem
    sh = "#htile.encoding<placement = shared>" if canonical else "#shared"
    lo = "#htile.encoding<placement = local>" if canonical else "#local"

    def t(shape, elt="f32", enc=None):
        enc = enc or lo
        return f"tensor<{'x'.join(str(d) for d in shape)}x{elt}, {enc}>"

    n = iter(range(1000))
    v = (lambda hint: f"%{next(n)}") if canonical else (lambda hint: f"%{hint}")
    zero_b = "%c0" if (canonical and grid[2] == 1) else "%bz"
    exp_op = "math.exp" if mutate == "exp" else "math.exp2"

    L = []
    if not canonical:
        L += ["#shared = #htile.encoding<placement = shared>",
              "#local = #htile.encoding<placement = local>", ""]
    L += ["module {",
          f"  func.func @{name}(%q: {mem}, %k: {kmem}, %v: {mem}, %out: {mem}) {{"]
    L += ["    %c0 = arith.constant 0 : index", "    %c1 = arith.constant 1 : index"]
    sizes = sorted({grid[0], grid[1], grid[2], threads, bm, bn, trip} - {0, 1})
    for s in sizes:
        L.append(f"    %c{s} = arith.constant {s} : index")
    cst0, cneg, cscale = ("%cst", "%cst_0", "%cst_1") if canonical else ("%f0", "%neg", "%scale")
    L += [f"    {cst0} = arith.constant 0.000000e+00 : f32",
          f"    {cneg} = arith.constant -3.40282347E+38 : f32",
          f"    {cscale} = arith.constant {scale!r} : f32"]

    def c(x):
        return "%c1" if x == 1 else f"%c{x}"

    L.append(f"    gpu.launch blocks(%bx, %by, %bz) in (%gx = {c(grid[0])}, %gy = {c(grid[1])}, "
             f"%gz = {c(grid[2])})")
    L.append(f"               threads(%tx, %ty, %tz) in (%sx = {c(threads)}, %sy = %c1, %sz = %c1) {{")
    ib, qs, m0, a0, s0 = v("i_base"), v("q_tile"), v("m0"), v("acc0"), v("l0")
    rowexpr = "%c0" if mutate == "q_row0" else ib
    L += [f"      {ib} = arith.muli %bx, {c(bm)} : index",
          f"      {qs} = htile.load %q[{zero_b}, %by, {rowexpr}, %c0] : {mem} -> {t([bm, D], e, sh)}",
          f"      {m0} = htile.full {cneg} : f32 -> {t([bm])}",
          f"      {a0} = htile.full {cst0} : f32 -> {t([bm, D])}",
          f"      {s0} = htile.full {cst0} : f32 -> {t([bm])}"]
    res = v("res") if canonical else None
    li, la, lm = v("l_i"), v("acc_i"), v("m_i")
    head = (f"{res}:3" if canonical else "%l_fin, %acc_fin, %m_fin")
    L.append(f"      {head} = scf.for %j = %c0 to {c(trip)} step %c1 "
             f"iter_args({li} = {s0}, {la} = {a0}, {lm} = {m0}) -> ({t([bm])}, {t([bm, D])}, {t([bm])}) {{")
    jb, kt, qk, sc, sco, rm, mn = (v(x) for x in ("j_base", "k_tile", "qk", "scale_t", "score",
                                                  "row_max", "m_next"))
    L.append(f"        {jb} = arith.muli %j, {c(bn)} : index")
    if k_mem == "ds":
        tb = " {transpose_b, warp_policy = \"full_row\"}" if mutate == "kt_transpose" else \
            " {warp_policy = \"full_row\"}"
        L.append(f"        {kt} = htile.load %k[{zero_b}, %by, %c0, {jb}] : {kmem} -> {t([D, bn], e, sh)}")
        L.append(f"        {qk} = htile.dot {qs}, {kt}{tb} : "
                 f"{t([bm, D], e, sh)}, {t([D, bn], e, sh)} -> {t([bm, bn])}")
    elif form == "pre":
        L.append(f"        {kt} = htile.load %k[{zero_b}, %by, {jb}, %c0] : {mem} -> {t([bn, D], e, sh)}")
        L.append(f"        {qk} = htile.dot {qs}, {kt} {{transpose_b, warp_policy = \"full_row\"}} : "
                 f"{t([bm, D], e, sh)}, {t([bn, D], e, sh)} -> {t([bm, bn])}")
    else:
        L.append(f"        {kt} = htile.load %k[{zero_b}, %by, {jb}, %c0] "
                 f"{{dimension_order = array<i64: 1, 0>}} : {mem} -> {t([D, bn], e, sh)}")
        L.append(f"        {qk} = htile.dot {qs}, {kt} {{warp_policy = \"full_row\"}} : "
                 f"{t([bm, D], e, sh)}, {t([D, bn], e, sh)} -> {t([bm, bn])}")
    L += [f"        {sc} = htile.full {cscale} : f32 -> {t([bm, bn])}",
          f"        {sco} = arith.mulf {qk}, {sc} : {t([bm, bn])}",
          f"        {rm} = htile.reduce {sco} axis 1 kind \"max\" : {t([bm, bn])} -> {t([bm])}",
          f"        {mn} = arith.maximumf {lm}, {rm} : {t([bm])}"]
    e64, b64, sh_, p, rs = (v(x) for x in ("e64", "b64", "shifted", "p", "row_sum"))
    L += [f"        {e64} = tensor.empty() : {t([bm, bn])}",
          f"        {b64} = linalg.broadcast ins({mn} : {t([bm])}) outs({e64} : {t([bm, bn])}) "
          f"dimensions = [1]",
          f"        {sh_} = arith.subf {sco}, {b64} : {t([bm, bn])}",
          f"        {p} = {exp_op} {sh_} : {t([bm, bn])}",
          f"        {rs} = htile.reduce {p} axis 1 kind \"sum\" : {t([bm, bn])} -> {t([bm])}"]
    d, ds, lsc, ln = (v(x) for x in ("dm", "dscale", "l_scaled", "l_next"))
    dm_expr = f"{mn}, {lm}" if mutate == "delta_sign" else f"{lm}, {mn}"
    L += [f"        {d} = arith.subf {dm_expr} : {t([bm])}",
          f"        {ds} = math.exp2 {d} : {t([bm])}",
          f"        {lsc} = arith.mulf {li}, {ds} : {t([bm])}",
          f"        {ln} = arith.addf {rs}, {lsc} : {t([bm])}" if canonical else
          f"        {ln} = arith.addf {lsc}, {rs} : {t([bm])}"]
    p16, vt, pv = v("p16"), v("v_tile"), v("pv")
    L += [f"        {p16} = arith.truncf {p} : {t([bm, bn])} to {t([bm, bn], e)}",
          f"        {vt} = htile.load %v[{zero_b}, %by, {jb}, %c0] : {mem} -> {t([bn, D], e, sh)}",
          f"        {pv} = htile.dot {p16}, {vt} {{warp_policy = \"full_row\"}} : {t([bm, bn], e)}, "
          f"{t([bn, D], e, sh)} -> {t([bm, D])}"]
    ea, ba, eb, bb, ad, asc, asd, an = (v(x) for x in ("ea", "bprev", "eb", "bnext", "adelta",
                                                      "ascale", "ascaled", "acc_next"))
    L += [f"        {ea} = tensor.empty() : {t([bm, D])}",
          f"        {ba} = linalg.broadcast ins({lm} : {t([bm])}) outs({ea} : {t([bm, D])}) dimensions = [1]",
          f"        {eb} = tensor.empty() : {t([bm, D])}",
          f"        {bb} = linalg.broadcast ins({mn} : {t([bm])}) outs({eb} : {t([bm, D])}) dimensions = [1]",
          f"        {ad} = arith.subf {ba}, {bb} : {t([bm, D])}",
          f"        {asc} = math.exp2 {ad} : {t([bm, D])}",
          f"        {asd} = arith.mulf {asc}, {la} : {t([bm, D])}" if canonical else
          f"        {asd} = arith.mulf {la}, {asc} : {t([bm, D])}"]
    if mutate == "no_rescale":
        L.append(f"        {an} = arith.addf {la}, {pv} : {t([bm, D])}")
    else:
        L.append(f"        {an} = arith.addf {asd}, {pv} : {t([bm, D])}")
    L.append(f"        scf.yield {ln}, {an}, {mn} : {t([bm])}, {t([bm, D])}, {t([bm])}")
    stage = f" {{htile.pipeline_stages = {stages} : i32}}" if stages is not None else ""
    L.append(f"      }}{stage}")
    lf, af = (f"{res}#0", f"{res}#1") if canonical else ("%l_fin", "%acc_fin")
    es, bs, nm, n16 = (v(x) for x in ("es", "bsum", "norm", "norm16"))
    L += [f"      {es} = tensor.empty() : {t([bm, D])}",
          f"      {bs} = linalg.broadcast ins({lf} : {t([bm])}) outs({es} : {t([bm, D])}) dimensions = [1]",
          f"      {nm} = arith.divf {af}, {bs} : {t([bm, D])}",
          f"      {n16} = arith.truncf {nm} : {t([bm, D])} to {t([bm, D], e)}",
          f"      htile.store {n16}, %out[{zero_b}, %by, {ib}, %c0] : {t([bm, D], e)}, {mem}",
          "      gpu.terminator",
          "    }",
          "    return",
          "  }",
          "}"]
    text = "\n".join(L) + "\n"
    if mutate == "unsupported":
        text = text.replace("math.exp2 %", "math.exp2x %", 1)
    return text
