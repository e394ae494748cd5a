'use strict';
/*
 * ewise_ref.js -- TEST INFRASTRUCTURE (the checker of q8_ewise), not product
 * code: only tests/ load it.
 *
 * A restatement of how the reference CPU backend turns an elementwise loop
 * nest into JavaScript (src/backend/cpu/codegen.ts:428-552 _exprToJS, the
 * operand folds, Math.fround on f32-typed MathOps and non-exact externs,
 * `| 0` casts; _flatIndex row-major offsets :548-551; dtype inference
 * src/compiler/ir/lir/nodes.ts:193-218; typed arrays src/util/dtype_map.ts:
 * 53-65).  The generated function runs in this Node process, so rounding,
 * Math.round, ToInt32 and typed-array stores are a real engine's.
 * Pinned by the expected strings of tests/backend/cpu/codegen-internals.test.js
 * (tests/node/ewise_test.js restates them as vectors).
 */

const INT = new Set(['i8', 'i16', 'i32', 'i64', 'ui8', 'index']);
const FLOAT = new Set(['f16', 'bf16', 'f32', 'f64']);
const ALIAS = { float32: 'f32', float64: 'f64', int32: 'i32', int8: 'i8', uint8: 'ui8', u8: 'ui8' };
const norm = (d) => ALIAS[d] || d;
const EXACT = new Set(['max', 'min', 'abs', 'floor', 'ceil', 'round', 'sign', 'sqrt', 'fmod']);
const JS_MATH = new Set(['exp', 'log', 'sqrt', 'tanh', 'abs', 'ceil', 'floor', 'sin', 'cos', 'max', 'min',
                         'pow', 'round', 'sign', 'log2', 'log10']);
const CMP = { eq: '===', ne: '!==', lt: '<', le: '<=', gt: '>', ge: '>=' };

function inferDtype(n) {
  if (!n) return 'f32';
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
      if (FLOAT.has(da)) return da;
      if (n.b) { const db = inferDtype(n.b); if (FLOAT.has(db)) return db; }
      return da;
    }
    case 'IfThenElseNode': return inferDtype(n.thenBody);
    default: return 'f32';
  }
}

const round = (dtype, e) => (dtype === 'f32' ? `Math.fround(${e})` : `(${e})`);

function exprToJS(n, aliases) {
  if (!n) return '0';
  switch (n.type) {
    case 'IntImmNode':
    case 'FloatImmNode': return String(n.value);
    case 'VariableNode': return (aliases && aliases.get(n.name)) || n.name;
    case 'BufferLoadNode': return `${n.buffer.name}[${flatIndex(n.buffer, n.indices, aliases)}]`;
    case 'MathOpNode': {
      if (!n.b) return `(${n.op}${exprToJS(n.a, aliases)})`;
      const a = exprToJS(n.a, aliases), b = exprToJS(n.b, aliases);
      const dtype = inferDtype(n);
      const foldsZero = INT.has(dtype) && (a === '0' || b === '0');
      if (n.op === '-' && b === '0') return a;
      if (n.op === '*' && b === '1') return a;
      if (n.op === '*' && a === '1') return b;
      if (foldsZero && n.op === '+') return b === '0' ? a : b;
      if (foldsZero && n.op === '*') return dtype === 'i64' ? '0n' : '0';
      if (n.op === '/' && INT.has(dtype)) return dtype === 'i64' ? `(${a} / ${b})` : `Math.trunc(${a} / ${b})`;
      if (n.op === '%') return `((${a} % ${b} + ${b}) % ${b})`;
      if (n.op === '//') return `Math.floor(${a} / ${b})`;
      if (n.op === 'tmod') return `(${a} % ${b})`;
      if (n.op === 'tdiv') return `((${a} / ${b}) | 0)`;
      return round(dtype, `${a} ${n.op} ${b}`);
    }
    case 'CompareNode': return `(${exprToJS(n.a, aliases)} ${CMP[n.direction]} ${exprToJS(n.b, aliases)})`;
    case 'IfThenElseNode':
      return `(${exprToJS(n.condition, aliases)} ? ${exprToJS(n.thenBody, aliases)} : ${exprToJS(n.elseBody, aliases)})`;
    case 'CastNode': {
      const inner = exprToJS(n.expr, aliases);
      if (n.toDtype === 'bool') return `(${inner} ? 1 : 0)`;
      if (INT.has(norm(n.toDtype))) return `(${inner} | 0)`;
      return `(+${inner})`;
    }
    case 'CallExternNode': {
      const args = n.args.map((x) => exprToJS(x, aliases)).join(', ');
      const name = n.externName;
      const dt = EXACT.has(name) ? '' : inferDtype(n);
      if (JS_MATH.has(name)) return EXACT.has(name) ? `Math.${name}(${args})` : round(dt, `Math.${name}(${args})`);
      if (name === 'rsqrt') return round(dt, `1.0 / Math.sqrt(${args})`);
      if (name === 'fmod') {
        const [a, b] = n.args.map((x) => exprToJS(x, aliases));
        return `((${a} % ${b} + ${b}) % ${b})`;
      }
      throw new Error(`CPU codegen: unsupported extern function "${name}"`);
    }
    default: throw new Error(`CPU codegen: unhandled expr node '${n.type}'`);
  }
}

// row-major flat index; a literal 0 index drops its term, one index is itself
function flatIndex(buffer, indices, aliases) {
  if (indices.length === 0) return '0';
  if (indices.length === 1) return exprToJS(indices[0], aliases);
  const terms = [];
  let stride = 1;
  const strides = new Array(indices.length);
  for (let d = indices.length - 1; d >= 0; d--) { strides[d] = stride; stride *= buffer.shape[d]; }
  for (let d = 0; d < indices.length; d++) {
    const e = exprToJS(indices[d], aliases);
    if (e === '0') continue;
    terms.push(strides[d] === 1 ? e : `${e} * ${strides[d]}`);
  }
  return terms.length ? terms.join(' + ') : '0';
}

/**
 * The JS function of an elementwise loop nest PrimFunc, taking the
 * parameters' typed arrays in bufferMap order.
 */
function compilePrimFunc(pf) {
  const params = [];
  for (const [, buf] of pf.bufferMap) params.push(buf);
  const aliases = new Map();
  const lines = [];
  let depth = 0;
  let n = pf.body;
  for (;;) {
    if (n.type === 'ForNode') {
      lines.push(`${'  '.repeat(depth)}for (let ${n.loopVar.name} = 0; ${n.loopVar.name} < ${exprToJS(n.extent)}; ${n.loopVar.name}++) {`);
      depth++;
      n = n.body;
    } else if (n.type === 'BlockNode') {
      for (const iv of n.iterVars || []) aliases.set(iv.iterVar.name, exprToJS(iv.binding, aliases));
      n = n.body;
    } else if (n.type === 'SeqNode' && n.stmts.length === 1) {
      n = n.stmts[0];
    } else if (n.type === 'LetStmtNode') {
      lines.push(`${'  '.repeat(depth)}const ${n.variable.name} = ${exprToJS(n.value, aliases)};`);
      n = n.body;
    } else {
      break;
    }
  }
  if (n.type !== 'BufferStoreNode') throw new Error('ewise_ref: not a single-store loop nest');
  let value = exprToJS(n.value, aliases);
  lines.push(`${'  '.repeat(depth)}${n.buffer.name}[${flatIndex(n.buffer, n.indices, aliases)}] = ${value};`);
  while (depth > 0) { depth--; lines.push(`${'  '.repeat(depth)}}`); }
  const src = `return function ${pf.name || 'kernel'}(${params.map((b) => b.name).join(', ')}) {\n${lines.join('\n')}\n};`;
  return { fn: new Function(src)(), source: src };
}

module.exports = { exprToJS, flatIndex, compilePrimFunc, inferDtype };
