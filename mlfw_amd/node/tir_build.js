'use strict';
/*
 * Builders of TIR PrimFuncs shaped like the ones the reference's
 * QuantizationPass and lowering rules produce: plain objects with the
 * reference's node field names (src/compiler/ir/tensor/nodes.ts), loop
 * nests built the way lowerPointwise builds them
 * (src/compiler/passes/lowering/lowering_registry.ts:277-306, 521-576:
 * loop vars i_d, block iter vars v_d bound to them, loads through
 * computeBroadcastIndices), the compiled quantize expression of
 * quant_math.ts:16-27 and the qmatmul init / accumulate blocks of
 * rules/quantization.ts:23-42.  Used where no reference compiler is at
 * hand: the tests and the plan benchmark (plan_bench.js).
 */
const V = (name, dtype = 'index') => ({ type: 'VariableNode', name, dtype });
const I = (value) => ({ type: 'IntImmNode', value });
const F = (value) => ({ type: 'FloatImmNode', value });
const buf = (name, shape, dtype) => ({ name, shape, dtype });
const load = (b, indices) => ({ type: 'BufferLoadNode', buffer: b, indices });
const math = (op, a, b = null) => ({ type: 'MathOpNode', op, a, b });
const ext = (externName, args, dtype = 'f32') => ({ type: 'CallExternNode', externName, args, dtype });
const cast = (expr, fromDtype, toDtype) => ({ type: 'CastNode', expr, fromDtype, toDtype });
const cmp = (direction, a, b) => ({ type: 'CompareNode', direction, a, b });
const sel = (condition, thenBody, elseBody) => ({ type: 'IfThenElseNode', condition, thenBody, elseBody });

let uid = 0;
function primFunc(name, params, body, consts) {
  const attrs = new Map();
  const bufferMap = new Map();
  params.forEach((b) => bufferMap.set(V(`p${uid++}`, 'handle'), b));
  if (consts && consts.length) attrs.set('const_buffers', consts);
  return {
    name, params: [...bufferMap.keys()], body, bufferMap, attrs,
    getAttr(k) { return attrs.has(k) ? attrs.get(k) : null; },
    setAttr(k, v) { attrs.set(k, v); return this; },
  };
}

/** lowerPointwise: loops over out's shape, loads through broadcast indices. */
function pointwise(name, out, inputs, exprBuilder, consts) {
  const n = out.shape.length, tag = uid++;
  const loopVars = [], ivs = [], indices = [];
  for (let d = 0; d < n; d++) {
    loopVars.push(V(`i${d}_${tag}`));
    const iv = V(`v${d}_${tag}`);
    ivs.push({ type: 'BlockRealizeNode', iterVar: iv, binding: loopVars[d], kind: 0 });
    indices.push(iv);
  }
  const loads = inputs.map((b) => {
    const off = n - b.shape.length;
    return load(b, b.shape.map((s, j) => (s === 1 ? I(0) : indices[off + j])));
  });
  const store = { type: 'BufferStoreNode', buffer: out, indices, value: exprBuilder(loads, indices) };
  let body = { type: 'BlockNode', name: `${name}_block`, iterVars: ivs, reads: inputs.map((b) => ({ buffer: b })),
               writes: [{ buffer: out }], body: store, initBody: null };
  for (let d = n - 1; d >= 0; d--) {
    body = { type: 'ForNode', loopVar: loopVars[d], min: I(0), extent: I(out.shape[d]), kind: 'serial', body };
  }
  const constBufs = (consts || []).map((c) => c.buffer);
  const params = inputs.filter((b) => !constBufs.includes(b)).concat([out], constBufs);
  return primFunc(name, params, body, consts);
}

/** quantize_block (quant_math.ts:16-27) around an inner expression. */
function quantizeExpr(e, scale, zp = 0, tgt = 'i8') {
  let s = math('/', e, F(scale));
  if (zp !== 0) s = math('+', s, F(zp));
  const lo = tgt === 'ui8' ? 0 : -128, hi = tgt === 'ui8' ? 255 : 127;
  return cast(ext('min', [ext('max', [ext('round', [s]), F(lo)]), F(hi)]), 'f32', tgt);
}

/** qmatmul_init / qmatmul_acc (rules/quantization.ts:23-42) with W [N,K]. */
function qmatmulPF(M, N, K, a, w, out, consts) {
  const tag = uid++;
  const m = V(`vm_${tag}`), n = V(`vn_${tag}`), k = V(`vk_${tag}`);
  const init = { type: 'BlockNode', name: 'qmatmul_init', iterVars: [], reads: [], writes: [{ buffer: out }],
                 body: { type: 'BufferStoreNode', buffer: out, indices: [m, n], value: I(0) } };
  const acc = { type: 'BlockNode', name: 'qmatmul_acc_1', iterVars: [], reads: [{ buffer: a }, { buffer: w }],
                writes: [{ buffer: out }],
                body: { type: 'BufferStoreNode', buffer: out, indices: [m, n],
                        value: math('+', load(out, [m, n]), math('*', cast(load(a, [m, k]), 'i8', 'i32'),
                                                               cast(load(w, [n, k]), 'i8', 'i32'))) } };
  return primFunc('qmatmul', [a, out, w], { type: 'ForNode', body: { type: 'SeqNode', stmts: [init, acc] } }, consts);
}


module.exports = { V, I, F, buf, load, math, ext, cast, cmp, sel, primFunc, pointwise, quantizeExpr, qmatmulPF };
