"""Site programs: the growth and pruning policies, traced for the device.

The reference calls a growth rule's ``propose`` / ``score`` / ``importance``
/ ``init`` and a PruneConn ``predicate`` under ``jax.vmap``, once per
proposal site, candidate pair, unit or edge (phases.py:3640-4058,
:1444-1498). Here each such callback is called once with symbolic views and
compiled to a *site program*: a register program over 32-bit values of four
kinds (float32, int32, uint32, bool) that the device interprets once per
site (``plx_site_prog`` in include/plastax_hip.h).

A site is described by up to five integer roles -- ``i`` (the proposing or
scored unit), ``j`` (the proposal index), ``src``, ``dst`` and ``cid`` (the
edge's arena slot) -- and, for proposals, by a Philox stream keyed as the
reference's ``Rng.for_site`` (rng.py:206-246): each ``uniform`` /
``uniform_int`` / ``bernoulli`` call reads the next sub-counter, fixed at
trace time exactly as the reference advances it.

Integer semantics follow jnp with 64-bit types off: int32 and uint32 wrap;
``//`` and ``%`` are floor division and floor modulo; ``astype`` from float
truncates toward zero and saturates (NaN goes to 0); ``/`` is float32 true
division.
"""

from __future__ import annotations

import dataclasses
from typing import Any, Sequence

import numpy as np

from plastax_amd._expr import (
    Expr,
    Index,
    UnsupportedPolicyError,
    binary,
    cast,
    kind_of_dtype,
    lift,
    unary,
)

# Site opcodes: keep in sync with plastax_amd/csrc/structural.hip and the
# oracle's evaluator (oracle/plastax_oracle.c).
SOP = {
    "const": 1, "idx": 2, "ldu": 3, "ldc": 4, "rng": 5, "mov": 6, "sel": 7, "out": 8,
    "fadd": 10, "fsub": 11, "fmul": 12, "fdiv": 13, "fneg": 14, "fabs": 15, "fmax": 16,
    "fmin": 17, "ftanh": 18, "fexp": 19, "flog": 20, "fsqrt": 21, "fsigmoid": 22,
    "fsquare": 23, "frelu": 24, "fsign": 25, "ffloor": 26, "fcos": 27, "fsin": 28,
    "fgt": 30, "fge": 31, "flt": 32, "fle": 33, "feq": 34, "fne": 35,
    "iadd": 40, "isub": 41, "imul": 42, "ineg": 43, "iabs": 44, "imax": 45, "imin": 46,
    "ifloordiv": 47, "imod": 48, "isign": 49,
    "igt": 50, "ige": 51, "ilt": 52, "ile": 53, "ieq": 54, "ine": 55,
    "umax": 60, "umin": 61, "ufloordiv": 62, "umod": 63, "ugt": 64, "uge": 65, "ult": 66,
    "ule": 67,
    "and": 70, "or": 71, "xor": 72, "not": 73, "shl": 74, "shru": 75, "shri": 76, "bnot": 77,
    "i2f": 80, "u2f": 81, "f2i": 82, "f2u": 83, "f2b": 84, "i2b": 85,
    "flog1p": 90, "fexpm1": 91,
}
ROLES = {"i": 0, "j": 1, "src": 2, "dst": 3, "cid": 4}
KIND_CODE = {"f": 0, "i": 1, "u": 2, "b": 3}
MAX_SREGS = 32
MAX_SINSTR = 160
MAX_SCONST = 32
MAX_SFIELDS = 8
MAX_SOUTS = 8


# ---------------------------------------------------------------------------
# Symbolic views of a site.
# ---------------------------------------------------------------------------


def idx(role: str) -> Expr:
    """The int32 value of one of the site's roles."""
    return Expr("idx", role=role, dtype="i")


def _index_expr(x: Any) -> Expr:
    if isinstance(x, Index):
        role = {"self": "i", "out": "i"}.get(x.role, x.role)
        return idx(role)
    e = lift(x)
    if e.dtype in ("f", "wf", "b"):
        raise UnsupportedPolicyError("a unit index must be an integer")
    return cast(e, np.int32) if e.dtype != "i" else e


class SiteUnitView:
    """``u[FIELD, idx]`` at any integer-valued index of the site."""

    def __init__(self, dtypes: dict[str, np.dtype]) -> None:
        self._dtypes = dtypes

    def __getitem__(self, key: tuple[Any, Any]) -> Expr:
        spec, at = key
        name = spec.name
        if name not in self._dtypes:
            raise UnsupportedPolicyError(f"unit field {name!r} is not a column of this net")
        return Expr("ldu", (_index_expr(at),), field=name, dtype=kind_of_dtype(self._dtypes[name]))

    def gather(self, spec: Any, ids: Any) -> Expr:
        return self[spec, ids]


class SiteConnView:
    """``c[FIELD, cid]`` at the site's own edge."""

    def __init__(self, dtypes: dict[str, np.dtype]) -> None:
        self._dtypes = dtypes

    def __getitem__(self, key: tuple[Any, Any]) -> Expr:
        spec, at = key
        if not (isinstance(at, Expr) and at.op == "idx" and at.role == "cid"):
            raise UnsupportedPolicyError("connection fields are read at the site's own cid")
        if spec.name not in self._dtypes:
            raise UnsupportedPolicyError(f"conn field {spec.name!r} is not a column of this net")
        return Expr("ldc", field=spec.name, role="cid", dtype=kind_of_dtype(self._dtypes[spec.name]))


class SiteGlobals:
    """``g["name"]`` / ``g.name``: a scalar global, refreshed per call."""

    def __init__(self, concrete: Any) -> None:
        self._concrete = concrete

    def _read(self, key: str) -> Expr:
        value = np.asarray(_read_global(self._concrete, key))
        return Expr("global", field=str(key), dtype=kind_of_dtype(value.dtype))

    def __getitem__(self, key: str) -> Expr:
        return self._read(key)

    def __getattr__(self, key: str) -> Expr:
        if key.startswith("_"):
            raise AttributeError(key)
        return self._read(key)


def _read_global(g: Any, name: str) -> Any:
    v = g[name] if isinstance(g, dict) else getattr(g, name)
    arr = np.asarray(v)
    if arr.shape != ():
        raise UnsupportedPolicyError(f"global {name!r} must be a scalar to be traced")
    return arr


class SiteRng:
    """The draw stream of one proposal site (rng.py:182-309): every call
    consumes the next sub-counter of ``philox32(site_seed, (j << 16) | sub)``."""

    def __init__(self) -> None:
        self._sub = 0

    def _draw(self) -> Expr:
        if self._sub >= 1 << 16:
            raise ValueError("Rng sub-counter exhausted (>= 2**16 draws)")
        e = Expr("rng", value=self._sub, dtype="u")
        self._sub += 1
        return e

    def uniform(self) -> Expr:
        """unit_float of the next word: float32(w >> 8) * 2^-24 (rng.py:144-153)."""
        w = self._draw()
        return cast(w >> 8, np.float32) * np.float32(1.0 / 16777216.0)

    def uniform_int(self, n: int) -> Expr:
        """min(uint32(uniform() * n), n - 1) (rng.py:273-287)."""
        n = int(n)
        if n < 1:
            raise ValueError("uniform_int needs n >= 1")
        scaled = cast(self.uniform() * np.float32(n), np.uint32)
        return binary("min", scaled, np.uint32(n - 1))

    def bernoulli(self, p: Any) -> Expr:
        """uniform() < p (rng.py:301-309)."""
        return binary("lt", self.uniform(), cast(lift(p), np.float32))

    def normal(self) -> Expr:
        """Box-Muller on the next two uniforms (rng.py:289-299):
        sqrt(-2 log(1 - u1)) * cos(2 pi u2), float32 throughout; log and cos
        are the framework's Cephes functions (within 2 ulp of the exact ones
        on Box-Muller's range), the same on the device and in the oracle."""
        u1 = self.uniform()
        u2 = self.uniform()
        r = unary("sqrt", binary("mul", np.float32(-2.0), unary("log", binary("sub", np.float32(1.0), u1))))
        return binary("mul", r, unary("cos", binary("mul", np.float32(6.28318530717958648), u2)))


# ---------------------------------------------------------------------------
# Compilation.
# ---------------------------------------------------------------------------


@dataclasses.dataclass
class SiteProgram:
    """A compiled site program (plx_site_prog)."""

    code: list[tuple[int, int, int, int]]
    consts: list[int]  # 32-bit patterns
    unit_fields: list[str]
    conn_fields: list[str]
    out_kinds: list[str]
    globals_at: dict[int, tuple[str, str]]  # const slot -> (global name, kind)
    draws: int  # rng sub-counters used

    @property
    def ninstr(self) -> int:
        return len(self.code)

    def flat_code(self) -> np.ndarray:
        return np.asarray(self.code, dtype=np.int32).reshape(-1)

    def const_bits(self, globals_: Any = None) -> np.ndarray:
        vals = np.asarray(self.consts, dtype=np.uint32).copy()
        for slot, (name, kind) in self.globals_at.items():
            vals[slot] = _bits(_read_global(globals_, name).item(), kind)
        return vals

    def uses_role(self, role: str) -> bool:
        return any(op == SOP["idx"] and a == ROLES[role] for op, _, a, _ in self.code)

    def const_output(self, k: int) -> int | None:
        """The int32 value of output k when the program writes a traced
        constant there (not a global, not a computed value); else None."""
        regs: dict[int, int] = {}  # register -> const slot it holds
        out: int | None = None
        written = False
        for op, d, a, _ in self.code:
            if op == SOP["out"]:
                if d == k:  # (the last write of the slot wins)
                    slot = regs.get(a)
                    written = True
                    out = None if slot is None or slot in self.globals_at else slot
                continue
            if op == SOP["const"]:
                regs[d] = a
            elif op == SOP["mov"] and a in regs:
                regs[d] = regs[a]
            else:
                regs.pop(d, None)
        if not written or out is None:
            return None
        return int(np.uint32(self.consts[out]).view(np.int32))


def _bits(value: Any, kind: str) -> int:
    if kind == "f":
        return int(np.float32(value).view(np.uint32))
    if kind == "b":
        return 1 if bool(value) else 0
    return int(value) & 0xFFFFFFFF  # int32 / uint32: two's complement bits


def _opcode(node: Expr) -> str:
    """The typed opcode of an arithmetic / comparison / logic node."""
    op, k = node.op, node.dtype
    arg_k = node.args[0].dtype if node.args else k
    cmp = {"gt", "ge", "lt", "le", "eq", "ne"}
    if op in cmp:
        if arg_k == "f":
            return "f" + op
        if arg_k == "u" and op in ("gt", "ge", "lt", "le"):
            return "u" + op
        return "i" + op  # int32, or eq/ne on any 32-bit pattern
    if op == "not":
        return "bnot" if k == "b" else "not"
    if op in ("and", "or", "xor"):
        return op
    if op == "shl":
        return "shl"
    if op == "shr":
        return "shru" if k == "u" else "shri"
    if k == "f":
        name = {"add": "fadd", "sub": "fsub", "mul": "fmul", "div": "fdiv", "neg": "fneg",
                "abs": "fabs", "max": "fmax", "min": "fmin", "tanh": "ftanh", "exp": "fexp",
                "log": "flog", "sqrt": "fsqrt", "sigmoid": "fsigmoid", "square": "fsquare",
                "relu": "frelu", "sign": "fsign", "floor": "ffloor", "cos": "fcos", "sin": "fsin",
                "log1p": "flog1p", "expm1": "fexpm1"}.get(op)
    elif k == "i":
        name = {"add": "iadd", "sub": "isub", "mul": "imul", "neg": "ineg", "abs": "iabs",
                "max": "imax", "min": "imin", "floordiv": "ifloordiv", "mod": "imod",
                "sign": "isign", "square": "imul"}.get(op)
    elif k == "u":
        name = {"add": "iadd", "sub": "isub", "mul": "imul", "neg": "ineg", "abs": None,
                "max": "umax", "min": "umin", "floordiv": "ufloordiv", "mod": "umod",
                "square": "imul"}.get(op)
    else:  # bool
        name = {"max": "or", "min": "and"}.get(op)
    if name is None:
        raise UnsupportedPolicyError(f"operation {op!r} on {k!r} values cannot run on the device")
    return name


def _cvt_ops(src: str, dst: str) -> list[str]:
    """The opcodes casting a value of kind ``src`` to ``dst`` (empty: same bits)."""
    if src == dst:
        return []
    table = {
        ("i", "f"): ["i2f"], ("u", "f"): ["u2f"], ("b", "f"): ["i2f"],
        ("f", "i"): ["f2i"], ("f", "u"): ["f2u"], ("f", "b"): ["f2b"],
        ("i", "u"): [], ("u", "i"): [], ("b", "i"): [], ("b", "u"): [],
        ("i", "b"): ["i2b"], ("u", "b"): ["i2b"],
    }
    return table[(src, dst)]


def compile_site_program(outputs: Sequence[tuple[Any, str]], *, roles: Sequence[str]) -> SiteProgram:
    """Compile ``(expr, kind)`` outputs to a site program. ``roles`` names the
    site roles the context defines; reading another raises."""
    allowed = set(roles)
    outs = [cast(lift(e), {"f": np.float32, "i": np.int32, "u": np.uint32, "b": np.bool_}[k])
            for e, k in outputs]
    if len(outs) > MAX_SOUTS:
        raise UnsupportedPolicyError(f"a policy writes {len(outs)} values; at most {MAX_SOUTS}")

    order: list[Expr] = []
    seen: set[int] = set()
    for o in outs:
        stack = [(o, False)]
        while stack:
            node, done = stack.pop()
            if id(node) in seen:
                continue
            if done:
                seen.add(id(node))
                order.append(node)
                continue
            stack.append((node, True))
            for a in reversed(node.args):
                if id(a) not in seen:
                    stack.append((a, False))

    last_use: dict[int, int] = {}
    for pos, node in enumerate(order):
        for a in node.args:
            last_use[id(a)] = pos
    for o in outs:
        last_use[id(o)] = len(order)

    consts: list[int] = []
    const_slot: dict[Any, int] = {}
    globals_at: dict[int, tuple[str, str]] = {}
    ufields: list[str] = []
    cfields: list[str] = []
    reg: dict[int, int] = {}
    free = list(range(MAX_SREGS - 1, -1, -1))
    code: list[tuple[int, int, int, int]] = []
    draws = 0

    def const_index(key: Any, bits: int) -> int:
        if key not in const_slot:
            if len(consts) >= MAX_SCONST:
                raise UnsupportedPolicyError("a policy uses too many constants")
            const_slot[key] = len(consts)
            consts.append(bits)
        return const_slot[key]

    def take() -> int:
        if not free:
            raise UnsupportedPolicyError("a policy expression needs too many registers")
        return free.pop()

    def field_slot(table: list[str], name: str) -> int:
        if name not in table:
            if len(table) >= MAX_SFIELDS:
                raise UnsupportedPolicyError("a policy reads too many fields")
            table.append(name)
        return table.index(name)

    for pos, node in enumerate(order):
        op = node.op
        k = node.dtype if node.dtype not in ("wi", "wf") else ("f" if node.dtype == "wf" else "i")
        pre: list[tuple[str, int, int]] = []  # (opcode, a, b) emitted into d
        if op == "const":
            bits = _bits(node.value, k)
            pre = [("const", const_index(("c", k, bits), bits), 0)]
        elif op == "global":
            slot = const_index(("g", node.field), 0)
            globals_at[slot] = (str(node.field), k)
            pre = [("const", slot, 0)]
        elif op == "idx":
            if node.role not in allowed:
                raise UnsupportedPolicyError(f"{node.role!r} is not defined for this policy")
            pre = [("idx", ROLES[node.role], 0)]
        elif op == "rng":
            if "rng" not in allowed:
                raise UnsupportedPolicyError("this policy has no rng")
            draws = max(draws, int(node.value) + 1)
            pre = [("rng", int(node.value), 0)]
        elif op == "ldu":
            pre = [("ldu", field_slot(ufields, str(node.field)), reg[id(node.args[0])])]
        elif op == "ldc":
            if "cid" not in allowed:
                raise UnsupportedPolicyError("connection fields are not visible to this policy")
            pre = [("ldc", field_slot(cfields, str(node.field)), 0)]
        elif op == "cvt":
            src_k = node.args[0].dtype
            ops = _cvt_ops(src_k, k)
            a = reg[id(node.args[0])]
            pre = [(o, a, 0) for o in ops] or [("mov", a, 0)]
            if len(pre) > 1:
                raise AssertionError("casts are one instruction")
        elif op == "sel":
            c, t, f = (reg[id(a)] for a in node.args)
            pair = _take_pair(free)
            code.append((SOP["mov"], pair, t, 0))
            code.append((SOP["mov"], pair + 1, f, 0))
            pre = [("sel", c, pair)]
        elif op == "relu" and k in ("i", "u"):
            zero = const_index(("c", k, 0), 0)
            z = take()
            code.append((SOP["const"], z, zero, 0))
            pre = [("imax" if k == "i" else "umax", reg[id(node.args[0])], z)]
            free.append(z)
        elif op == "square" and k in ("i", "u"):
            a = reg[id(node.args[0])]
            pre = [("imul", a, a)]
        elif len(node.args) == 1:
            pre = [(_opcode(node), reg[id(node.args[0])], 0)]
        elif len(node.args) == 2:
            pre = [(_opcode(node), reg[id(node.args[0])], reg[id(node.args[1])])]
        else:
            raise UnsupportedPolicyError(f"operation {op!r} cannot run on the device")
        for a in node.args:
            if last_use.get(id(a)) == pos and reg[id(a)] not in free:
                free.append(reg[id(a)])
        d = take()
        reg[id(node)] = d
        name, a0, b0 = pre[0]
        code.append((SOP[name], d, a0, b0))
        if op == "sel":
            free.append(b0)
            free.append(b0 + 1)
    for slot, o in enumerate(outs):
        code.append((SOP["out"], slot, reg[id(o)], 0))
    if len(code) > MAX_SINSTR:
        raise UnsupportedPolicyError(f"a policy compiles to {len(code)} instructions; at most {MAX_SINSTR}")
    return SiteProgram(code, consts, ufields, cfields, [k for _, k in outputs], globals_at, draws)


def _take_pair(free: list[int]) -> int:
    s = set(free)
    for r in range(0, MAX_SREGS - 1):
        if r in s and r + 1 in s:
            free.remove(r)
            free.remove(r + 1)
            return r
    raise UnsupportedPolicyError("a policy expression needs too many registers")


# ---------------------------------------------------------------------------
# Tracing the growth and pruning callbacks.
# ---------------------------------------------------------------------------


def _triple(out: Any) -> tuple[Any, Any, Any]:
    if hasattr(out, "src") and hasattr(out, "dst") and hasattr(out, "score"):
        return out.src, out.dst, out.score
    src, dst, score = out
    return src, dst, score


def trace_propose(rule: Any, proposer: str, unit_dtypes: dict, conn_dtypes: dict, g: Any) -> SiteProgram:
    """ProposeAddConn.propose for one site -> (src i32, dst i32, score f32)
    (phases.py:3766-3860, :3921-4038)."""
    u = SiteUnitView(unit_dtypes)
    rng = SiteRng()
    gg = SiteGlobals(g)
    if proposer == "per_unit":
        out = rule.propose(u, idx("i"), idx("j"), gg, rng)
        roles = ("i", "j", "rng")
    elif proposer == "per_connection":
        c = SiteConnView(conn_dtypes)
        out = rule.propose(u, c, idx("cid"), idx("j"), gg, rng)
        roles = ("cid", "j", "rng")
    elif proposer == "global":
        out = rule.propose(u, idx("j"), gg, rng)
        roles = ("j", "rng")
    else:
        raise ValueError(f"unknown proposer {proposer!r}")
    src, dst, score = _triple(out)
    return compile_site_program([(src, "i"), (dst, "i"), (score, "f")], roles=roles)


def trace_score(rule: Any, unit_dtypes: dict, g: Any) -> SiteProgram:
    """ScoreAddConn.score(u, src, dst, g) -> f32 (phases.py:4771-4774)."""
    out = rule.score(SiteUnitView(unit_dtypes), idx("src"), idx("dst"), SiteGlobals(g))
    return compile_site_program([(out, "f")], roles=("src", "dst"))


def trace_importance(rule: Any, unit_dtypes: dict, g: Any) -> SiteProgram:
    """importance(u, i, g) -> f32 (phases.py:3640-3665)."""
    out = rule.importance(SiteUnitView(unit_dtypes), idx("i"), SiteGlobals(g))
    return compile_site_program([(out, "f")], roles=("i",))


def trace_init(rule: Any, unit_dtypes: dict, conn_specs: Sequence[Any], g: Any) -> tuple[SiteProgram, list[str]]:
    """init(u, src, dst, g) -> ConnWrite; returns the program and the conn
    field each output slot writes (phases.py:4776-4781, :4979-5005)."""
    write = rule.init(SiteUnitView(unit_dtypes), idx("src"), idx("dst"), SiteGlobals(g))
    fields = dict(getattr(write, "fields", write))
    specs = {s.name: s for s in conn_specs}
    outs, names = [], []
    for name, value in fields.items():
        if name not in specs:
            raise UnsupportedPolicyError(f"init writes {name!r}, which is not a conn column")
        if name in ("from_id", "to_id", "dead"):
            continue  # the claim writes these itself
        outs.append((value, kind_of_dtype(specs[name].dtype)))
        names.append(name)
    return compile_site_program(outs, roles=("src", "dst")), names


def trace_conn_update(fn: Any, direction: str, unit_dtypes: dict, conn_specs: Sequence[Any],
                      g: Any) -> tuple[SiteProgram, list[str]]:
    """One pass of a user UpdateConn (sweep.py:488-532) as an edge program:
    ``incoming(u, dst, src, c, cid, g)`` or ``outgoing(u, src, dst, c, cid,
    g)`` -> ConnWrite, each written column merged keep-old on dead rows
    (``where(dead, old, new)``, sweep.py:527-529). Returns the program and the
    column each output writes. Writes of FROM_ID / TO_ID / DEAD (structure)
    and of columns narrower than 32 bits are refused."""
    specs = {s.name: s for s in conn_specs}
    conn_dtypes = {n: np.dtype(s.dtype) for n, s in specs.items()}
    u, c, gv = SiteUnitView(unit_dtypes), SiteConnView(conn_dtypes), SiteGlobals(g)
    cid = idx("cid")
    if direction == "incoming":
        write = fn(u, idx("dst"), idx("src"), c, cid, gv)
    else:
        write = fn(u, idx("src"), idx("dst"), c, cid, gv)
    fields = dict(getattr(write, "fields", write))
    dead = c[_Field("dead"), cid]
    outs, names = [], []
    for name, value in fields.items():
        if name not in specs:
            raise UnsupportedPolicyError(f"update_conn writes {name!r}, which is not a conn column")
        if name in ("from_id", "to_id", "dead"):
            raise UnsupportedPolicyError(f"update_conn may not write {name!r} (the arena's structure)")
        if conn_dtypes[name].itemsize != 4:
            raise UnsupportedPolicyError(f"update_conn writes {name!r}, a {conn_dtypes[name]} column: "
                                         "the device writes 32-bit connection columns")
        kind = kind_of_dtype(conn_dtypes[name])
        outs.append((_select(dead, c[_Field(name), cid], value, kind), kind))
        names.append(name)
    return compile_site_program(outs, roles=("cid", "src", "dst")), names


class _Field:
    """A column name in the shape of a FieldSpec (for the views)."""

    def __init__(self, name: str) -> None:
        self.name = name


def _select(cond: Expr, a: Any, b: Any, kind: str) -> Expr:
    ty = {"f": np.float32, "i": np.int32, "u": np.uint32, "b": np.bool_}[kind]
    return Expr("sel", (cast(cond, np.bool_), cast(lift(a), ty), cast(lift(b), ty)), dtype=kind)


def trace_predicate(rule: Any, unit_dtypes: dict, conn_dtypes: dict, g: Any) -> SiteProgram:
    """PruneConn.predicate(u, c, cid, g) -> bool (phases.py:1444-1498)."""
    out = rule.predicate(SiteUnitView(unit_dtypes), SiteConnView(conn_dtypes), idx("cid"), SiteGlobals(g))
    return compile_site_program([(out, "b")], roles=("cid", "src", "dst"))



def _unit_outputs(write: Any, unit_dtypes: dict) -> tuple[list[tuple[Any, str]], list[str]]:
    fields = dict(getattr(write, "fields", write))
    outs, names = [], []
    for name, value in fields.items():
        if name not in unit_dtypes:
            raise UnsupportedPolicyError(f"a unit policy writes {name!r}, which is not a unit column")
        outs.append((value, kind_of_dtype(unit_dtypes[name])))
        names.append(name)
    return outs, names


def trace_update_unit(rule: Any, unit_dtypes: dict, g: Any) -> tuple[SiteProgram, list[str]]:
    """UpdateUnit.update(u, i, g) -> UnitWrite (phases.py:1148-1193)."""
    write = rule.update(SiteUnitView(unit_dtypes), idx("i"), SiteGlobals(g))
    outs, names = _unit_outputs(write, unit_dtypes)
    return compile_site_program(outs, roles=("i",)), names


def trace_prune_unit(rule: Any, unit_dtypes: dict, g: Any) -> SiteProgram:
    """PruneUnit.predicate(u, i, g) -> bool (phases.py:1245-1307)."""
    out = rule.predicate(SiteUnitView(unit_dtypes), idx("i"), SiteGlobals(g))
    return compile_site_program([(out, "b")], roles=("i",))


class _Pruned:
    name = "pruned"


def trace_spawn(rule: Any, unit_dtypes: dict, g: Any) -> SiteProgram:
    """AddUnit.spawn(u, parent, g) -> (spawns bool, level offset int32)
    (phases.py:1362-1367); the first output is already "a live unit that
    spawns"."""
    u = SiteUnitView(unit_dtypes)
    wants, offset = rule.spawn(u, idx("i"), SiteGlobals(g))
    wants = cast(lift(wants), np.bool_)
    if "pruned" in unit_dtypes:
        # a parent is a live unit that spawns (phases.py:1374)
        wants = binary("and", wants, binary("eq", cast(u[_Pruned, idx("i")], np.int32), 0))
    return compile_site_program([(wants, "b"), (offset, "i")], roles=("i",))


def trace_unit_init(rule: Any, unit_dtypes: dict, g: Any) -> tuple[SiteProgram, list[str]]:
    """AddUnit.init(u, child, parent, g) -> UnitWrite (phases.py:1398-1405);
    the child is the site's src role and the parent its dst role."""
    write = rule.init(SiteUnitView(unit_dtypes), idx("src"), idx("dst"), SiteGlobals(g))
    outs, names = _unit_outputs(write, unit_dtypes)
    return compile_site_program(outs, roles=("src", "dst")), names


def trace_pass_map(policy: Any, backward: bool, unit_dtypes: dict, conn_dtypes: dict,
                   g: Any) -> SiteProgram:
    """A forward or backward pass's ``map`` outside the product form, as an
    edge program with one float32 output per accumulator component
    (sweep.py:113-180 / :343-399): forward ``map(u, dst, src, c, cid, g)``,
    backward ``map(u, src, dst, c, cid, g)``; a tuple map is one output per
    element."""
    u, c, gv = SiteUnitView(unit_dtypes), SiteConnView(conn_dtypes), SiteGlobals(g)
    if backward:
        out = policy.map(u, idx("src"), idx("dst"), c, idx("cid"), gv)
    else:
        out = policy.map(u, idx("dst"), idx("src"), c, idx("cid"), gv)
    comps = list(out) if isinstance(out, tuple) else [out]
    outs = []
    for k, e in enumerate(comps):
        e = lift(e)
        if e.dtype not in ("f", "wf"):
            raise UnsupportedPolicyError(
                f"{type(policy).__name__}.map: component {k} is not float32 (generic passes accumulate float32)")
        outs.append((e, "f"))
    return compile_site_program(outs, roles=("cid", "src", "dst"))


def acc_field_names(k: int) -> list[str]:
    """The unit columns a generic pass's apply reads its accumulator from."""
    return [f"__acc{j}" for j in range(k)]


def trace_pass_apply(policy: Any, ncomp: int, tuple_acc: bool, unit_dtypes: dict,
                     g: Any) -> tuple[SiteProgram, list[str]]:
    """A generic pass's ``apply(u, i, g, acc)`` -> UnitWrite as a unit
    program; the accumulator (a tuple when ``tuple_acc``) is read from the
    unit columns ``acc_field_names(ncomp)``."""
    names = acc_field_names(ncomp)
    acc_view = SiteUnitView({n: np.dtype(np.float32) for n in names})
    comps = [acc_view[_Field(n), idx("i")] for n in names]
    acc = tuple(comps) if tuple_acc else comps[0]
    write = policy.apply(SiteUnitView(unit_dtypes), idx("i"), SiteGlobals(g), acc)
    outs, written = _unit_outputs(write, unit_dtypes)
    return compile_site_program(outs, roles=("i",)), written
