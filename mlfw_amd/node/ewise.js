'use strict';
/*
 * ewise.js -- translate an elementwise TIR PrimFunc into the device program
 * of q8_ewise (include/q8hip.h).
 *
 * Accepted form: the loop nest lowerPointwise / the fused 'inline-loop'
 * lowering builds (src/compiler/passes/lowering/lowering_registry.ts:277-306,
 * 564-576; rules/fusion.ts): serial ForNodes with constant extents starting
 * at 0, BlockNodes whose iter vars are bound to (affine expressions of) the
 * loop variables, optional LetStmtNode bindings, and one BufferStoreNode whose
 * indices are the loop nest's own indices in order.  Loads may use any
 * affine index (broadcasts: the computeBroadcastIndices forms, :521-538).
 *
 * The value expression is compiled with the reference CPU codegen's rules
 * (src/backend/cpu/codegen.ts:428-552, dtype inference
 * src/compiler/ir/lir/nodes.ts:193-218): the same operand folds ('x - 0',
 * 'x * 1', integer '+ 0' / '* 0'), Math.fround on f32-typed arithmetic and
 * non-exact externs, no rounding on exact externs, `| 0` for casts to an
 * integer type.  Anything outside that subset returns null and the
 * PrimFunc keeps its normal codegen.
 */

const Q8_I8 = 0, Q8_U8 = 1, Q8_I32 = 2, Q8_F32 = 3, Q8_F64 = 4;
const MAX_DIMS = 6, MAX_INPUTS = 8, MAX_CODE = 96, MAX_REGS = 16, MAX_CONST = 32;

const OP = {
  LOAD: 0, CONST: 1, INDEX: 2, ADD: 3, SUB: 4, MUL: 5, DIV: 6, IDIV: 7, MOD: 8, FLOORDIV: 9,
  TMOD: 10, TDIV: 11, NEG: 12, CMP: 13, SELECT: 14, TOINT32: 15, TOBOOL: 16, MAX: 17, MIN: 18,
  ABS: 19, FLOOR: 20, CEIL: 21, ROUND: 22, SIGN: 23, SQRT: 24, FMOD: 25, EXP: 26, LOG: 27,
  TANH: 28, RSQRT: 29, POW: 30,
};
const CMP_DIR = { eq: 0, ne: 1, lt: 2, le: 3, gt: 4, ge: 5 };
const ARITH = { '+': OP.ADD, '-': OP.SUB, '*': OP.MUL, '/': OP.DIV };
const EXACT_EXTERNS = { max: OP.MAX, min: OP.MIN, abs: OP.ABS, floor: OP.FLOOR, ceil: OP.CEIL,
                        round: OP.ROUND, sign: OP.SIGN, sqrt: OP.SQRT, fmod: OP.FMOD };
const ROUNDED_EXTERNS = { exp: OP.EXP, log: OP.LOG, tanh: OP.TANH, rsqrt: OP.RSQRT, pow: OP.POW };

const DTYPE_ALIAS = { float32: 'f32', float64: 'f64', int32: 'i32', int8: 'i8', uint8: 'ui8', u8: 'ui8' };
const norm = (d) => DTYPE_ALIAS[d] || d;
const INT_DTYPES = new Set(['i8', 'i16', 'i32', 'i64', 'ui8', 'index']);
const FLOAT_DTYPES = new Set(['f16', 'bf16', 'f32', 'f64']);
const isInt = (d) => INT_DTYPES.has(norm(d));
const isFloat = (d) => FLOAT_DTYPES.has(norm(d));
const ELEM = { i8: Q8_I8, ui8: Q8_U8, bool: Q8_U8, i32: Q8_I32, index: Q8_I32, f32: Q8_F32, f64: Q8_F64 };

class Reject extends Error {}
function need(c, why) { if (!c) throw new Reject(why); }

// inferDtype (src/compiler/ir/lir/nodes.ts:193-218)
function inferDtype(n) {
  if (!n) return 'f32';
  if (n._dtype) return norm(n._dtype);
  switch (n.type) {
    case 'IntImmNode': return 'i32';
    case 'FloatImmNode': return 'f32';
    case 'BufferLoadNode': return norm(n.buffer.dtype);
    case 'CastNode': return norm(n.toDtype);
    case 'CallExternNode': return norm(n.dtype || 'f32');
    case 'CompareNode': return 'i32';
    case 'VariableNode': return norm(n.dtype || 'i32');
    case 'MathOpNode': {
      const da = inferDtype(n.a);
      if (isFloat(da)) return da;
      if (n.b) { const db = inferDtype(n.b); if (isFloat(db)) return db; }
      return da;
    }
    case 'IfThenElseNode': return inferDtype(n.thenBody);
    default: return 'f32';
  }
}

// Affine form {coef: Map(dim -> k), c} of an index expression over the loop
// dims; `env` resolves iter vars and let vars to their expressions.
function affine(e, env) {
  if (!e) return null;
  if (e.type === 'IntImmNode') return { coef: new Map(), c: e.value };
  if (e.type === 'VariableNode') {
    if (env.loopDim.has(e.name)) return { coef: new Map([[env.loopDim.get(e.name), 1]]), c: 0 };
    const bound = env.iter.get(e.name) || env.lets.get(e.name);
    return bound ? affine(bound, env) : null;
  }
  if (e.type !== 'MathOpNode' || !e.b) return null;
  const a = affine(e.a, env), b = affine(e.b, env);
  if (!a || !b) return null;
  if (e.op === '+' || e.op === '-') {
    const s = e.op === '+' ? 1 : -1;
    const coef = new Map(a.coef);
    for (const [d, k] of b.coef) coef.set(d, (coef.get(d) || 0) + s * k);
    return { coef, c: a.c + s * b.c };
  }
  if (e.op === '*') {
    if (a.coef.size === 0) return { coef: new Map([...b.coef].map(([d, k]) => [d, k * a.c])), c: a.c * b.c };
    if (b.coef.size === 0) return { coef: new Map([...a.coef].map(([d, k]) => [d, k * b.c])), c: a.c * b.c };
  }
  return null;
}

function flatAffine(buffer, indices, env) {
  const shape = buffer.shape;
  need(Array.isArray(shape) && shape.every((d) => typeof d === 'number'), 'dynamic buffer shape');
  need(indices.length === shape.length, 'index rank');
  const coef = new Array(MAX_DIMS + 1).fill(0);
  let stride = 1;
  for (let d = shape.length - 1; d >= 0; d--) {
    const f = affine(indices[d], env);
    need(f, 'non-affine index');
    for (const [dim, k] of f.coef) coef[dim] += k * stride;
    coef[MAX_DIMS] += f.c * stride;
    stride *= shape[d];
  }
  return { coef, numel: stride };
}

/**
 * Translate a PrimFunc.  Returns { prog, inputIdx: [param index per input],
 * outIdx, ninputs, outNumel, inNumel } or null when the PrimFunc is not an
 * elementwise loop nest of the supported form.
 */
function translateEwise(primFunc) {
  try { return translate(primFunc); } catch (e) { if (e instanceof Reject) return null; throw e; }
}

function translate(primFunc) {
  const env = { loopDim: new Map(), iter: new Map(), lets: new Map() };
  const extents = [];
  let n = primFunc.body;
  for (;;) {
    need(n, 'empty body');
    if (n.type === 'ForNode') {
      need(n.min && n.min.type === 'IntImmNode' && n.min.value === 0, 'loop min');
      need(n.extent && n.extent.type === 'IntImmNode', 'dynamic extent');
      need(!n.threadTag, 'thread-bound loop');
      need(extents.length < MAX_DIMS, 'too many loops');
      env.loopDim.set(n.loopVar.name, extents.length);
      extents.push(n.extent.value);
      n = n.body;
    } else if (n.type === 'BlockNode') {
      need(!n.initBody, 'reduction block');
      for (const iv of n.iterVars || []) env.iter.set(iv.iterVar.name, iv.binding);
      n = n.body;
    } else if (n.type === 'SeqNode' && n.stmts && n.stmts.length === 1) {
      n = n.stmts[0];
    } else if (n.type === 'LetStmtNode') {
      env.lets.set(n.variable.name, n.value);
      n = n.body;
    } else {
      break;
    }
  }
  need(n.type === 'BufferStoreNode', 'not a single store');
  const out = n.buffer;
  need(out.shape.length === extents.length && out.shape.every((d, i) => d === extents[i]), 'store shape');
  for (let d = 0; d < n.indices.length; d++) {
    const f = affine(n.indices[d], env);
    need(f && f.c === 0 && f.coef.size === 1 && f.coef.get(d) === 1, 'store index is not the loop index');
  }
  const outDtype = ELEM[norm(out.dtype)];
  need(outDtype !== undefined, 'output dtype');

  const params = [];
  for (const [, buf] of primFunc.bufferMap) params.push(buf);
  const paramIndex = (buf) => params.findIndex((b) => b === buf || b.name === buf.name);
  const outIdx = paramIndex(out);
  need(outIdx >= 0, 'output is not a parameter');

  // ---- expression -> SSA code
  const code = [];            // {op, dst, a, b, c, aux, rnd}; dst/a/b/c are virtual registers
  const konst = [];
  const inputs = [];          // {param, dtype, coef, numel}
  const memo = new Map();     // node -> {v, lit}
  const letMemo = new Map();
  let nv = 0;
  const emit = (ins) => { need(code.length < MAX_CODE, 'program too long'); ins.dst = nv++; code.push(ins); return ins.dst; };
  const constVal = (value) => {
    let k = konst.findIndex((x) => Object.is(x, value));
    if (k < 0) { need(konst.length < MAX_CONST, 'too many constants'); konst.push(value); k = konst.length - 1; }
    return emit({ op: OP.CONST, aux: k });
  };

  // returns {v: virtual register, lit: printed literal or null}
  function expr(e) {
    need(e, 'null expression');
    if (memo.has(e)) return memo.get(e);
    const r = exprUncached(e);
    memo.set(e, r);
    return r;
  }
  function exprUncached(e) {
    switch (e.type) {
      case 'IntImmNode':
      case 'FloatImmNode':
        need(typeof e.value === 'number', 'immediate');
        return { v: constVal(e.value), lit: String(e.value) };
      case 'VariableNode': {
        if (env.loopDim.has(e.name)) return { v: emit({ op: OP.INDEX, aux: env.loopDim.get(e.name) }), lit: null };
        if (env.iter.has(e.name)) return expr(env.iter.get(e.name));
        if (env.lets.has(e.name)) {
          if (!letMemo.has(e.name)) letMemo.set(e.name, expr(env.lets.get(e.name)));
          return letMemo.get(e.name);
        }
        throw new Reject('free variable');
      }
      case 'BufferLoadNode': {
        const buf = e.buffer;
        const dt = ELEM[norm(buf.dtype)];
        need(dt !== undefined, 'load dtype');
        const p = paramIndex(buf);
        need(p >= 0 && p !== outIdx, 'load of a non-parameter or of the output');
        const { coef, numel } = flatAffine(buf, e.indices, env);
        let j = inputs.findIndex((x) => x.param === p && x.coef.every((c, i) => c === coef[i]));
        if (j < 0) { need(inputs.length < MAX_INPUTS, 'too many inputs'); inputs.push({ param: p, dtype: dt, coef, numel }); j = inputs.length - 1; }
        return { v: emit({ op: OP.LOAD, aux: j }), lit: null };
      }
      case 'MathOpNode': {
        if (!e.b) {
          need(e.op === '-', 'unary operator');
          const a = expr(e.a);
          return { v: emit({ op: OP.NEG, a: a.v }), lit: null };
        }
        const a = expr(e.a), b = expr(e.b);
        const dtype = inferDtype(e);
        const foldsZero = isInt(dtype) && (a.lit === '0' || b.lit === '0');
        if (e.op === '-' && b.lit === '0') return a;
        if (e.op === '*' && b.lit === '1') return a;
        if (e.op === '*' && a.lit === '1') return b;
        if (foldsZero && e.op === '+') return b.lit === '0' ? a : b;
        need(norm(dtype) !== 'i64', 'i64 arithmetic');
        if (foldsZero && e.op === '*') return { v: constVal(0), lit: '0' };
        if (e.op === '/' && isInt(dtype)) return { v: emit({ op: OP.IDIV, a: a.v, b: b.v }), lit: null };
        if (e.op === '%') return { v: emit({ op: OP.MOD, a: a.v, b: b.v }), lit: null };
        if (e.op === '//') return { v: emit({ op: OP.FLOORDIV, a: a.v, b: b.v }), lit: null };
        if (e.op === 'tmod') return { v: emit({ op: OP.TMOD, a: a.v, b: b.v }), lit: null };
        if (e.op === 'tdiv') return { v: emit({ op: OP.TDIV, a: a.v, b: b.v }), lit: null };
        const op = ARITH[e.op];
        need(op !== undefined, `operator ${e.op}`);
        return { v: emit({ op, a: a.v, b: b.v, rnd: dtype === 'f32' ? 1 : 0 }), lit: null };
      }
      case 'CompareNode': {
        need(CMP_DIR[e.direction] !== undefined, 'compare direction');
        const a = expr(e.a), b = expr(e.b);
        return { v: emit({ op: OP.CMP, a: a.v, b: b.v, aux: CMP_DIR[e.direction] }), lit: null };
      }
      case 'IfThenElseNode': {
        need(e.elseBody, 'select without else');
        const c = expr(e.condition), t = expr(e.thenBody), f = expr(e.elseBody);
        return { v: emit({ op: OP.SELECT, a: c.v, b: t.v, c: f.v }), lit: null };
      }
      case 'CastNode': {
        const x = expr(e.expr);
        const to = norm(e.toDtype);
        if (to === 'bool') return { v: emit({ op: OP.TOBOOL, a: x.v }), lit: null };
        need(to !== 'f16' && to !== 'bf16', 'half cast');
        if (isInt(to)) return { v: emit({ op: OP.TOINT32, a: x.v }), lit: null };
        return { v: x.v, lit: null };                       // (+x)
      }
      case 'CallExternNode': {
        const name = e.externName;
        const args = e.args.map(expr);
        if (EXACT_EXTERNS[name] !== undefined) {
          const binary = name === 'max' || name === 'min' || name === 'fmod';
          need(args.length === (binary ? 2 : 1), `arity of ${name}`);
          return { v: emit({ op: EXACT_EXTERNS[name], a: args[0].v, b: binary ? args[1].v : 0 }), lit: null };
        }
        need(ROUNDED_EXTERNS[name] !== undefined, `extern ${name}`);
        need(args.length === (name === 'pow' ? 2 : 1), `arity of ${name}`);
        const rnd = inferDtype(e) === 'f32' ? 1 : 0;
        return { v: emit({ op: ROUNDED_EXTERNS[name], a: args[0].v, b: name === 'pow' ? args[1].v : 0, rnd }), lit: null };
      }
      default:
        throw new Reject(`node ${e.type}`);
    }
  }

  const result = expr(n.value);
  // ---- register allocation: virtual -> one of MAX_REGS LDS registers
  const lastUse = new Array(nv).fill(-1);
  code.forEach((ins, i) => {
    for (const k of ['a', 'b', 'c']) if (usesOperand(ins, k)) lastUse[ins[k]] = i;
  });
  lastUse[result.v] = code.length;
  const phys = new Array(nv).fill(-1);
  const free = [];
  for (let r = MAX_REGS - 1; r >= 0; r--) free.push(r);
  const out8 = [];
  code.forEach((ins, i) => {
    const mapped = { op: ins.op, a: 0, b: 0, c: 0, aux: ins.aux || 0, rnd: ins.rnd || 0, dst: 0 };
    for (const k of ['a', 'b', 'c']) if (usesOperand(ins, k)) mapped[k] = phys[ins[k]];
    // operands whose last use is this instruction free their register first
    for (const k of ['a', 'b', 'c']) {
      if (usesOperand(ins, k) && lastUse[ins[k]] === i && phys[ins[k]] >= 0) {
        free.push(phys[ins[k]]);
        phys[ins[k]] = -2;
      }
    }
    need(free.length > 0, 'more than 16 live values');
    phys[ins.dst] = free.pop();
    mapped.dst = phys[ins.dst];
    if (lastUse[ins.dst] < 0) { free.push(phys[ins.dst]); }   // dead value
    out8.push(mapped);
  });
  need(phys[result.v] >= 0, 'result register');

  const ssa = { code: code.map((c) => Object.assign({}, c)), konst: konst.slice(), result: result.v };
  const prog = {
    ndims: extents.length, ninputs: inputs.length, extent: extents.slice(),
    inDtype: inputs.map((x) => x.dtype), inCoef: inputs.map((x) => x.coef), outDtype,
    ncode: out8.length, result: phys[result.v], nconst: konst.length, code: out8, konst: konst.slice(),
  };
  return { prog, ssa, inputs: inputs.map((x) => ({ param: x.param, dtype: x.dtype, coef: x.coef })),
           inputIdx: inputs.map((x) => x.param), inNumel: inputs.map((x) => x.numel),
           outIdx, outNumel: extents.reduce((a, b) => a * b, 1) };
}

/**
 * Recognises the per-channel epilogue group QuantizationPass leaves after a
 * quantized_dot (quantization_pass.ts:431-456: convert -> broadcast -> mul by
 * the f32 scale vector sv[n]), optionally followed by the layer's bias add,
 * ReLU (maximum with a broadcast zero, builder.ts:561-565) and the next
 * layer's static `quantize` (quant_math.ts:16-27, zero point 0, int8):
 *   out[m,n] = [Q]( [max]( [fround(] fround((+acc[m,n]) * sv[n]) [+ b[n])] [, 0)] )
 * on a 2-D [M, N] nest.  `isZero(param)` tells whether a parameter is a
 * constant buffer holding only +0.  Returns the roles of the inputs or null.
 */
function matchEpilogue(tr, isZero) {
  if (!tr || tr.prog.ndims !== 2) return null;
  const [M, N] = tr.prog.extent;
  const def = new Map(tr.ssa.code.map((c) => [c.dst, c]));
  const konst = tr.ssa.konst;
  const isConst = (v, x) => { const c = def.get(v); return c && c.op === OP.CONST && Object.is(konst[c.aux], x); };
  const constOf = (v) => { const c = def.get(v); return c && c.op === OP.CONST ? konst[c.aux] : undefined; };
  const load = (v) => { const c = def.get(v); return c && c.op === OP.LOAD ? tr.inputs[c.aux] : null; };
  const isRow = (inp) => inp && inp.coef[0] === 0 && inp.coef[1] === 1 && inp.coef[6] === 0;      // x[n]
  const isFull = (inp) => inp && inp.coef[0] === N && inp.coef[1] === 1 && inp.coef[6] === 0;     // x[m, n]
  let cur = tr.ssa.result;
  const out = { M, N, quant: null, relu: false, biasParam: -1, svParam: -1, accParam: -1 };
  if (tr.prog.outDtype === Q8_I8) {
    const c1 = def.get(cur);                       // Cast(.., i8) -> `| 0`
    if (!c1 || c1.op !== OP.TOINT32) return null;
    const mn = def.get(c1.a);
    if (!mn || mn.op !== OP.MIN || !isConst(mn.b, 127)) return null;
    const mx = def.get(mn.a);
    if (!mx || mx.op !== OP.MAX || !isConst(mx.b, -128)) return null;
    const rd = def.get(mx.a);
    if (!rd || rd.op !== OP.ROUND) return null;
    const dv = def.get(rd.a);
    const s = dv ? constOf(dv.b) : undefined;
    if (!dv || dv.op !== OP.DIV || !dv.rnd || typeof s !== 'number' || !(s > 0) || !isFinite(s)) return null;
    out.quant = { scale: s };
    cur = dv.a;
  } else if (tr.prog.outDtype !== Q8_F32) {
    return null;
  }
  let c = def.get(cur);
  if (c && c.op === OP.MAX) {
    const zeroArg = (v) => isConst(v, 0) || (load(v) && isZero(load(v).param));
    if (zeroArg(c.b)) { out.relu = true; cur = c.a; } else if (zeroArg(c.a)) { out.relu = true; cur = c.b; } else return null;
    c = def.get(cur);
  }
  if (c && c.op === OP.ADD) {
    if (!c.rnd) return null;
    const bb = load(c.b), ba = load(c.a);
    if (isRow(bb) && bb.dtype === Q8_F32) { out.biasParam = bb.param; cur = c.a; }
    else if (isRow(ba) && ba.dtype === Q8_F32) { out.biasParam = ba.param; cur = c.b; }
    else return null;
    c = def.get(cur);
  }
  if (!c || c.op !== OP.MUL || !c.rnd) return null;
  for (const [accV, svV] of [[c.a, c.b], [c.b, c.a]]) {
    const acc = load(accV), sv = load(svV);
    if (isFull(acc) && acc.dtype === Q8_I32 && isRow(sv) && sv.dtype === Q8_F32) {
      out.accParam = acc.param;
      out.svParam = sv.param;
      return out;
    }
  }
  return null;
}

function usesOperand(ins, k) {
  const op = ins.op;
  if (op === OP.LOAD || op === OP.CONST || op === OP.INDEX) return false;
  if (k === 'a') return true;
  if (k === 'b') {
    return !(op === OP.NEG || op === OP.TOINT32 || op === OP.TOBOOL || op === OP.ABS || op === OP.FLOOR ||
             op === OP.CEIL || op === OP.ROUND || op === OP.SIGN || op === OP.SQRT || op === OP.EXP ||
             op === OP.LOG || op === OP.TANH || op === OP.RSQRT);
  }
  return op === OP.SELECT;
}

// ---- binary layout of q8_ew_prog (natural C alignment, include/q8hip.h)
const LAYOUT = (() => {
  let o = 0;
  const f = {};
  f.ndims = o; o += 4;
  f.ninputs = o; o += 4;
  f.extent = o; o += 8 * MAX_DIMS;
  f.inDtype = o; o += 4 * MAX_INPUTS;
  f.inCoef = o; o += 8 * MAX_INPUTS * (MAX_DIMS + 1);
  f.outDtype = o; o += 4;
  f.ncode = o; o += 4;
  f.result = o; o += 4;
  f.nconst = o; o += 4;
  f.code = o; o += 8 * MAX_CODE;
  o = (o + 7) & ~7;
  f.konst = o; o += 8 * MAX_CONST;
  f.bytes = o;
  return f;
})();

/** Pack a translated program into the bytes of a q8_ew_prog. */
function packProg(p) {
  const buf = new ArrayBuffer(LAYOUT.bytes);
  const dv = new DataView(buf);
  const i32 = (off, v) => dv.setInt32(off, v, true);
  const i64 = (off, v) => {
    need(Number.isSafeInteger(v), 'coefficient');
    dv.setInt32(off, v | 0, true);   // low word (two's complement)
    dv.setInt32(off + 4, Math.floor(v / 4294967296), true);
  };
  i32(LAYOUT.ndims, p.ndims);
  i32(LAYOUT.ninputs, p.ninputs);
  for (let d = 0; d < p.ndims; d++) i64(LAYOUT.extent + 8 * d, p.extent[d]);
  for (let j = 0; j < p.ninputs; j++) {
    i32(LAYOUT.inDtype + 4 * j, p.inDtype[j]);
    for (let d = 0; d <= MAX_DIMS; d++) i64(LAYOUT.inCoef + 8 * ((MAX_DIMS + 1) * j + d), p.inCoef[j][d]);
  }
  i32(LAYOUT.outDtype, p.outDtype);
  i32(LAYOUT.ncode, p.ncode);
  i32(LAYOUT.result, p.result);
  i32(LAYOUT.nconst, p.nconst);
  p.code.forEach((ins, i) => {
    const o = LAYOUT.code + 8 * i;
    [ins.op, ins.dst, ins.a, ins.b, ins.c, ins.aux, ins.rnd, 0].forEach((v, k) => dv.setUint8(o + k, v));
  });
  p.konst.forEach((v, k) => dv.setFloat64(LAYOUT.konst + 8 * k, v, true));
  return new Uint8Array(buf);
}

module.exports = { translateEwise, matchEpilogue, packProg, inferDtype, LAYOUT, OP, ELEM,
                   Q8_I8, Q8_U8, Q8_I32, Q8_F32, Q8_F64 };
