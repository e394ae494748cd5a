'use strict';
/*
 * hip_backend.js -- the MI355X int8 path behind mlfw's own plugin surfaces.
 *
 * registerHip(registries) plugs three things into a running mlfw, using the
 * registry functions the reference exports:
 *   1. runtime backend 'hip' (registerBackend, src/runtime/backend_registry.ts:14-32):
 *      RuntimeModule.run/runAsync (src/runtime/runtime.ts:261-275) dispatch on
 *      kernel.metadata.kind and hand the kernel's typed arrays to runSync;
 *   2. external codegen 'hip_int8' (registerExternalCodegen,
 *      src/backend/codegen_registry.ts:17-36) and its provider
 *      (registerExternalCodegenProvider, src/compiler/pipeline/external_codegen.ts:11-35):
 *      annotate() tags the PrimFuncs that QuantizationPass's ops lower to
 *      (`quantize`, `dequantize`, `quantized_dot`, `quantized_conv`; block names from
 *      src/compiler/passes/lowering/rules/quantization.ts and
 *      lowering_registry.ts:313,329,574) and compile() returns a descriptor
 *      instead of source, the pattern of the cuBLAS entry
 *      (codegen_registry.ts:46-52);
 *   3. an eager dispatcher library 'q8' (Library(ns).def().impl(),
 *      src/dispatcher/library.ts:30-72) with the dynamic per-token ops.
 * Every op runs on the GPU through the addon; nothing falls back to the CPU.
 */

const HIP_KIND = 'hip';
const PROVIDER = 'hip_int8';

let _q8 = null;
function q8() {
  if (!_q8) _q8 = require('./index.js');
  return _q8;
}

// ---------------------------------------------------------------- TIR matching
function collectBlocks(primFunc) {
  const blocks = [];
  const stack = [primFunc.body];
  while (stack.length > 0) {
    const n = stack.pop();
    if (!n) continue;
    if (n.type === 'BlockNode') { blocks.push(n); stack.push(n.body); continue; }
    if (n.body) stack.push(n.body);
    if (n.stmts) for (const s of n.stmts) stack.push(s);
    if (n.thenBody) stack.push(n.thenBody);
    if (n.elseBody) stack.push(n.elseBody);
  }
  return blocks;
}

function findStore(node) {
  const stack = [node];
  while (stack.length > 0) {
    const n = stack.pop();
    if (!n) continue;
    if (n.type === 'BufferStoreNode') return n;
    if (n.body) stack.push(n.body);
    if (n.stmts) for (const s of n.stmts) stack.push(s);
  }
  return null;
}

function numel(shape) {
  let n = 1;
  for (const d of shape) {
    if (typeof d !== 'number') return null;
    n *= d;
  }
  return n;
}

function paramIndex(primFunc, buffer) {
  const names = [];
  for (const [, buf] of primFunc.bufferMap) names.push(buf.name);
  return names.indexOf(buffer.name);
}

const INT8_DTYPES = new Set(['i8', 'ui8']);
const isImm = (n) => n && (n.type === 'FloatImmNode' || n.type === 'IntImmNode');
const isExtern = (n, name) => n && n.type === 'CallExternNode' && n.externName === name;
const isMath = (n, op) => n && n.type === 'MathOpNode' && n.op === op;

// quant_math.ts:16-27: Cast(min(max(round((x / s) [+ zp]), cMin), cMax))
function matchQuantizeExpr(e) {
  if (!e || e.type !== 'CastNode') return null;
  const mn = e.expr;
  if (!isExtern(mn, 'min') || !isImm(mn.args[1])) return null;
  const mx = mn.args[0];
  if (!isExtern(mx, 'max') || !isImm(mx.args[1])) return null;
  const rd = mx.args[0];
  if (!isExtern(rd, 'round')) return null;
  let scaled = rd.args[0];
  let zeroPoint = 0;
  if (isMath(scaled, '+') && isImm(scaled.b)) { zeroPoint = scaled.b.value; scaled = scaled.a; }
  if (!isMath(scaled, '/') || !isImm(scaled.b) || !scaled.a || scaled.a.type !== 'BufferLoadNode') return null;
  return { scale: scaled.b.value, zeroPoint, targetDtype: e.toDtype, clampMin: mx.args[1].value,
           clampMax: mn.args[1].value, load: scaled.a };
}

// quant_math.ts:29-34: ((+q) [- zp]) * s
function matchDequantizeExpr(e) {
  if (!isMath(e, '*') || !isImm(e.b)) return null;
  let shifted = e.a;
  let zeroPoint = 0;
  if (isMath(shifted, '-') && isImm(shifted.b)) { zeroPoint = shifted.b.value; shifted = shifted.a; }
  if (!shifted || shifted.type !== 'CastNode' || !shifted.expr || shifted.expr.type !== 'BufferLoadNode') return null;
  return { scale: e.b.value, zeroPoint, load: shifted.expr };
}

function varsIn(node, out) {
  const stack = [node];
  while (stack.length > 0) {
    const n = stack.pop();
    if (!n) continue;
    if (n.type === 'VariableNode') out.add(n.name);
    for (const k of ['a', 'b', 'expr']) if (n[k]) stack.push(n[k]);
    if (n.args) for (const a of n.args) stack.push(a);
    if (n.indices) for (const a of n.indices) stack.push(a);
  }
  return out;
}

function findLoad(node, buffer) {
  const stack = [node];
  while (stack.length > 0) {
    const n = stack.pop();
    if (!n) continue;
    if (n.type === 'BufferLoadNode' && n.buffer.name === buffer.name) return n;
    for (const k of ['a', 'b', 'expr', 'value', 'condition', 'thenBody', 'elseBody']) if (n[k]) stack.push(n[k]);
    if (n.args) for (const a of n.args) stack.push(a);
  }
  return null;
}

// An index expression as sum(coef * var) + const, or null when it is not
// linear (floor division, modulo, loads).  mathOp folds x*1 and x+0
// (src/compiler/ir/tensor/nodes.ts:394-430), so the forms vary.
function linearize(e) {
  if (!e) return null;
  if (e.type === 'IntImmNode') return { coef: new Map(), c: e.value };
  if (e.type === 'VariableNode') return { coef: new Map([[e.name, 1]]), c: 0 };
  if (e.type !== 'MathOpNode') return null;
  const a = linearize(e.a), b = linearize(e.b);
  if (!a || !b) return null;
  if (e.op === '+' || e.op === '-') {
    const sg = e.op === '+' ? 1 : -1;
    const coef = new Map(a.coef);
    for (const [v, k] of b.coef) coef.set(v, (coef.get(v) || 0) + sg * k);
    return { coef, c: a.c + sg * b.c };
  }
  if (e.op === '*') {
    if (a.coef.size === 0) return { coef: new Map([...b.coef].map(([v, k]) => [v, k * a.c])), c: a.c * b.c };
    if (b.coef.size === 0) return { coef: new Map([...a.coef].map(([v, k]) => [v, k * b.c])), c: a.c * b.c };
  }
  return null;
}

// qconv_acc of buildConvNest (src/compiler/passes/lowering/lowering_registry.ts:
// 335-449): out[n, oc, o..] += guard(in[n, c(oc, ic), o*stride + k*dil - lo], ker[oc, ic, k..]).
// Strides, dilation and leading padding are the coefficients and constant
// of each input spatial index; the trailing padding only fixes the output
// size, so the smallest one that gives the output's shape is used.
function detectConv(blocks, primFunc) {
  const init = blocks.find((b) => b.name.startsWith('qconv_init'));
  const acc = blocks.find((b) => b.name.startsWith('qconv_acc'));
  if (!init || !acc || acc.reads.length !== 2 || acc.writes.length !== 1) return null;
  const X = acc.reads[0].buffer, W = acc.reads[1].buffer, Y = acc.writes[0].buffer;
  if (!INT8_DTYPES.has(X.dtype) || !INT8_DTYPES.has(W.dtype) || Y.dtype !== 'i32') return null;
  const r = X.shape.length, d = r - 2;
  if (d < 1 || d > 3 || W.shape.length !== r || Y.shape.length !== r) return null;
  if (![...X.shape, ...W.shape, ...Y.shape].every((v) => typeof v === 'number')) return null;
  if (X.shape[1] % W.shape[1] !== 0) return null;
  const groups = X.shape[1] / W.shape[1];
  if (W.shape[0] % groups !== 0 || Y.shape[0] !== X.shape[0] || Y.shape[1] !== W.shape[0]) return null;
  const store = findStore(acc.body);
  if (!store || store.indices.length !== r) return null;
  const xl = findLoad(store.value, X), wl = findLoad(store.value, W);
  if (!xl || !wl) return null;
  const outVar = (i) => (store.indices[i].type === 'VariableNode' ? store.indices[i].name : null);
  const kerVar = (i) => (wl.indices[i].type === 'VariableNode' ? wl.indices[i].name : null);
  const strides = [], padLo = [], padHi = [], dilation = [];
  for (let s = 0; s < d; s++) {
    const S = X.shape[2 + s], K = W.shape[2 + s], P = Y.shape[2 + s];
    const lin = linearize(xl.indices[2 + s]);
    if (!lin) return null;
    const ov = outVar(2 + s), kv = kerVar(2 + s);
    for (const v of lin.coef.keys()) if (v !== ov && v !== kv) return null;
    // a dimension of extent 1 may have its variable folded away
    const st = ov ? (lin.coef.get(ov) || 0) : 0, dl = kv ? (lin.coef.get(kv) || 0) : 0;
    const stride = P === 1 && st === 0 ? 1 : st, dil = K === 1 && dl === 0 ? 1 : dl;
    if (stride < 1 || dil < 1 || lin.c > 0) return null;
    const lo = 0 - lin.c, eff = (K - 1) * dil + 1;   // 0 - 0 is +0
    const hi = Math.max(0, (P - 1) * stride + eff - S - lo);
    if (Math.floor((S + lo + hi - eff) / stride) + 1 !== P) return null;
    strides.push(stride); padLo.push(lo); padHi.push(hi); dilation.push(dil);
  }
  const product = isMath(store.value, '+') ? store.value.b : null;
  const inner = product && product.type === 'IfThenElseNode' ? product.thenBody : product;
  const zpX = inner && isMath(inner, '*') ? zeroPointOf(inner, X) : 0;
  const zpW = inner && isMath(inner, '*') ? zeroPointOf(inner, W) : 0;
  const xIdx = paramIndex(primFunc, X), wIdx = paramIndex(primFunc, W), outIdx = paramIndex(primFunc, Y);
  if (xIdx < 0 || wIdx < 0 || outIdx < 0) return null;
  return { op: 'quantized_conv', d, xShape: X.shape.slice(), wShape: W.shape.slice(),
           outShape: Y.shape.slice(), strides, padLo, padHi, dilation, groups, zpX, zpW,
           xDtype: X.dtype, wDtype: W.dtype, xIdx, wIdx, outIdx, outputIndices: [outIdx] };
}

// acc += ((a|0) [- zpA]) * ((b|0) [- zpB])  (rules/quantization.ts:33-39)
function zeroPointOf(product, buffer) {
  for (const side of [product.a, product.b]) {
    if (isMath(side, '-') && isImm(side.b) && findLoad(side.a, buffer)) return side.b.value;
    if (findLoad(side, buffer)) return 0;
  }
  return 0;
}

/**
 * Returns the hip_int8 descriptor of a PrimFunc that is exactly one int8
 * op of the quantized path, or null.
 */
function detectInt8Kernel(primFunc) {
  const blocks = collectBlocks(primFunc);
  if (blocks.length === 1 && /^(de)?quantize_block/.test(blocks[0].name)) {
    const b = blocks[0];
    const store = findStore(b.body);
    if (!store || b.reads.length !== 1 || b.writes.length !== 1) return null;
    const inBuf = b.reads[0].buffer, outBuf = b.writes[0].buffer;
    const n = numel(outBuf.shape);
    if (n === null || numel(inBuf.shape) !== n) return null;       // no broadcasting here
    const inIdx = paramIndex(primFunc, inBuf), outIdx = paramIndex(primFunc, outBuf);
    if (inIdx < 0 || outIdx < 0) return null;
    if (b.name.startsWith('quantize_block')) {
      const m = matchQuantizeExpr(store.value);
      if (!m || inBuf.dtype !== 'f32' || (outBuf.dtype !== 'i8' && outBuf.dtype !== 'ui8')) return null;
      return { op: 'quantize', n, scale: m.scale, zeroPoint: m.zeroPoint, targetDtype: outBuf.dtype,
               inIdx, outIdx, outputIndices: [outIdx] };
    }
    const m = matchDequantizeExpr(store.value);
    if (!m || outBuf.dtype !== 'f32' || ['i8', 'ui8', 'i32'].indexOf(inBuf.dtype) < 0) return null;
    return { op: 'dequantize', n, scale: m.scale, zeroPoint: m.zeroPoint, srcDtype: inBuf.dtype,
             inIdx, outIdx, outputIndices: [outIdx] };
  }
  if (blocks.length === 2 && blocks.some((b) => b.name.startsWith('qconv_acc'))) {
    return detectConv(blocks, primFunc);
  }
  if (blocks.length === 2) {
    const init = blocks.find((b) => b.name.startsWith('qmatmul_init'));
    const acc = blocks.find((b) => b.name.startsWith('qmatmul_acc'));
    if (!init || !acc || acc.reads.length !== 2 || acc.writes.length !== 1) return null;
    const A = acc.reads[0].buffer, B = acc.reads[1].buffer, C = acc.writes[0].buffer;
    // the verifier's QUANTIZED_INT_DTYPES (ops/quantization.ts:141-146)
    if (!INT8_DTYPES.has(A.dtype) || !INT8_DTYPES.has(B.dtype) || C.dtype !== 'i32') return null;
    if (A.shape.length !== 2 || B.shape.length !== 2 || C.shape.length !== 2) return null;
    const [M, K] = A.shape, N = C.shape[1];
    if (C.shape[0] !== M || ![M, N, K].every((d) => typeof d === 'number')) return null;
    const store = findStore(acc.body);
    if (!store) return null;
    // the contracting dim of B is the index that uses the reduction
    // variable (the one absent from the output's indices)
    const outVars = varsIn({ indices: store.indices }, new Set());
    const bLoad = findLoad(store.value, B);
    if (!bLoad) return null;
    const redPos = bLoad.indices.findIndex((ix) => {
      const vs = varsIn(ix, new Set());
      for (const v of vs) if (!outVars.has(v)) return true;
      return false;
    });
    let rhsLayout;
    if (redPos === 0 && B.shape[0] === K && B.shape[1] === N) rhsLayout = 'KN';
    else if (redPos === 1 && B.shape[0] === N && B.shape[1] === K) rhsLayout = 'NK';
    else return null;
    const product = isMath(store.value, '+') ? store.value.b : null;
    const zpA = product ? zeroPointOf(product, A) : 0;
    const zpB = product ? zeroPointOf(product, B) : 0;
    const aIdx = paramIndex(primFunc, A), bIdx = paramIndex(primFunc, B), outIdx = paramIndex(primFunc, C);
    if (aIdx < 0 || bIdx < 0 || outIdx < 0) return null;
    return { op: 'quantized_dot', M, N, K, rhsLayout, zpA, zpB, aDtype: A.dtype, bDtype: B.dtype,
             aIdx, bIdx, outIdx, outputIndices: [outIdx] };
  }
  return null;
}

// ---------------------------------------------------------------- runtime backend
const SRC_CODE = { i8: 'Q8_I8', ui8: 'Q8_U8', i32: 'Q8_I32' };
const ACT_CODE = { none: 'Q8_ACT_NONE', relu: 'Q8_ACT_RELU', silu: 'Q8_ACT_SILU' };

function bytesOf(a) { return a.byteLength; }

/** Device buffers of one kernel instance, reused across runs. */
class DeviceArgs {
  constructor() { this.bufs = new Map(); }
  get(key, bytes) {
    let b = this.bufs.get(key);
    if (!b || q8().bytes(b) < bytes) {
      if (b) q8().free(b);
      b = q8().alloc(Math.max(bytes, 1));
      this.bufs.set(key, b);
    }
    return b;
  }
  release() {
    for (const b of this.bufs.values()) q8().free(b);
    this.bufs.clear();
  }
}

function need(cond, msg) {
  if (!cond) throw new Error(`hip backend: ${msg}`);
}

function transposeI8(b, rows, cols) {
  const t = new Int8Array(rows * cols);
  for (let r = 0; r < rows; r++) for (let c = 0; c < cols; c++) t[c * rows + r] = b[r * cols + c];
  return t;
}

function f64(v) { return new Float64Array([v]); }

/** Runs one descriptor on typed arrays (host in, host out, device in between). */
function runDescriptor(d, args, dev) {
  const A = q8();
  if (d.op === 'quantize') {
    const x = args[d.inIdx], q = args[d.outIdx];
    need(x instanceof Float32Array && x.length === d.n, 'quantize input must be a Float32Array of n');
    need(q.length === d.n && (q instanceof Int8Array || q instanceof Uint8Array), 'quantize output');
    const dx = dev.get('x', bytesOf(x)), dq = dev.get('q', d.n);
    A.upload(dx, x);
    A.quantizeStatic(dx, d.n, d.scale, d.zeroPoint, A[d.targetDtype === 'ui8' ? 'Q8_U8' : 'Q8_I8'], dq);
    A.download(q, dq);
    return q;
  }
  if (d.op === 'dequantize') {
    const q = args[d.inIdx], y = args[d.outIdx];
    need(q.length === d.n && y instanceof Float32Array && y.length === d.n, 'dequantize shapes');
    const dq = dev.get('q', bytesOf(q)), ds = dev.get('s', 8), dy = dev.get('y', 4 * d.n);
    A.upload(dq, q);
    A.upload(ds, f64(d.scale));
    A.dequantize(dq, A[SRC_CODE[d.srcDtype]], 1, d.n, ds, A.Q8_PER_TENSOR, d.zeroPoint, dy);
    A.download(y, dy);
    return y;
  }
  if (d.op === 'quantized_dot') {
    const a = args[d.aIdx], b = args[d.bIdx], out = args[d.outIdx];
    const aT = (d.aDtype || 'i8') === 'ui8' ? Uint8Array : Int8Array;
    const bT = (d.bDtype || 'i8') === 'ui8' ? Uint8Array : Int8Array;
    need(a instanceof aT && a.length === d.M * d.K, 'quantized_dot lhs');
    need(b instanceof bT && b.length === d.N * d.K, 'quantized_dot rhs');
    need(out instanceof Int32Array && out.length === d.M * d.N, 'quantized_dot output');
    const aD = aT === Uint8Array ? A.Q8_U8 : A.Q8_I8, bD = bT === Uint8Array ? A.Q8_U8 : A.Q8_I8;
    const da = dev.get('a', d.M * d.K), db = dev.get('b', d.N * d.K), dout = dev.get('out', 4 * d.M * d.N);
    const wsBytes = A.quantizedDotWorkspace(d.M, d.N, d.K, aD, bD, d.zpA, d.zpB);
    const dws = wsBytes > 0 ? dev.get('ws', wsBytes) : null;
    A.upload(da, a);
    A.upload(db, d.rhsLayout === 'KN' ? transposeI8(b, d.K, d.N) : b);
    // zero points and ui8 operands: the exact correction inside the call
    A.quantizedDot(da, aD, db, bD, d.M, d.N, d.K, d.zpA, d.zpB, dws, dout);
    A.download(out, dout);
    return out;
  }
  if (d.op === 'quantized_conv') {
    const x = args[d.xIdx], w = args[d.wIdx], out = args[d.outIdx];
    const nx = numel(d.xShape), nw = numel(d.wShape), ny = numel(d.outShape);
    const xT = (d.xDtype || 'i8') === 'ui8' ? Uint8Array : Int8Array;
    const wT = (d.wDtype || 'i8') === 'ui8' ? Uint8Array : Int8Array;
    need(x instanceof xT && x.length === nx, 'quantized_conv input');
    need(w instanceof wT && w.length === nw, 'quantized_conv kernel');
    need(out instanceof Int32Array && out.length === ny, 'quantized_conv output');
    const wsBytes = A.convWorkspace(d.d, d.xShape, d.wShape, d.strides, d.padLo, d.padHi, d.dilation, d.groups);
    const dx = dev.get('x', nx), dw = dev.get('w', nw), dout = dev.get('out', 4 * ny);
    const dws = wsBytes > 0 ? dev.get('ws', wsBytes) : null;
    A.upload(dx, x);
    A.upload(dw, w);
    A.quantizedConvEx(dx, xT === Uint8Array ? A.Q8_U8 : A.Q8_I8, dw, wT === Uint8Array ? A.Q8_U8 : A.Q8_I8,
                      d.d, d.xShape, d.wShape, d.strides, d.padLo, d.padHi, d.dilation, d.groups,
                      d.zpX, d.zpW, A.Q8_I32, 0, dws, dout);
    A.download(out, dout);
    return out;
  }
  if (d.op === 'qlinear') {
    // dynamic per-token int8 linear: x fp32 [M,K]; wq int8 [N,K] + f64 scales [N]
    const x = args[d.xIdx], wq = args[d.wqIdx], ws = args[d.wsIdx], out = args[d.outIdx];
    const bias = d.biasIdx === undefined || d.biasIdx < 0 ? null : args[d.biasIdx];
    need(x instanceof Float32Array && x.length === d.M * d.K, 'qlinear x');
    need(wq instanceof Int8Array && wq.length === d.N * d.K, 'qlinear wq');
    need(ws instanceof Float64Array && ws.length === d.N, 'qlinear weight scales');
    need(out instanceof Float32Array && out.length === d.M * d.N, 'qlinear out');
    need(bias === null || (bias instanceof Float32Array && bias.length === d.N), 'qlinear bias');
    const perTensor = d.granularity === 'per_tensor';
    const dx = dev.get('x', 4 * d.M * d.K), dxq = dev.get('xq', d.M * d.K);
    const dsx = dev.get('sx', 8 * (perTensor ? 1 : d.M));
    const dwq = dev.get('wq', d.N * d.K), dws = dev.get('ws', 8 * d.N);
    const db = bias ? dev.get('bias', 4 * d.N) : null, dout = dev.get('out', 4 * d.M * d.N);
    A.upload(dx, x);
    A.upload(dwq, wq);
    A.upload(dws, ws);
    if (bias) A.upload(db, bias);
    // quantize + GEMM + epilogue in one call (one kernel for a single token)
    A.qlinearDynamic(dx, d.M, d.K, perTensor ? A.Q8_PER_TENSOR : A.Q8_PER_TOKEN, dwq, dws, A.Q8_PER_CHANNEL,
                     d.N, db, A[ACT_CODE[d.act || 'none']], dout, dxq, dsx);
    A.download(out, dout);
    return out;
  }
  if (d.op === 'qlinear_requant') {
    // int8 linear whose output is requantized with the next layer's static
    // scale (the calibrated chain ... mul(sv) -> add(b) -> max -> quantize):
    // xq int8 [M,K] + f64 scale(s), wq int8 [N,K] + f64 scales [N] -> int8 [M,N]
    const xq = args[d.xqIdx], sx = args[d.sxIdx], wq = args[d.wqIdx], ws = args[d.wsIdx];
    const out = args[d.outIdx];
    const bias = d.biasIdx === undefined || d.biasIdx < 0 ? null : args[d.biasIdx];
    const perTensor = d.granularity === 'per_tensor';
    need(xq instanceof Int8Array && xq.length === d.M * d.K, 'qlinear_requant xq');
    need(sx instanceof Float64Array && sx.length === (perTensor ? 1 : d.M), 'qlinear_requant activation scales');
    need(wq instanceof Int8Array && wq.length === d.N * d.K, 'qlinear_requant wq');
    need(ws instanceof Float64Array && ws.length === d.N, 'qlinear_requant weight scales');
    need(out instanceof Int8Array && out.length === d.M * d.N, 'qlinear_requant out');
    need(bias === null || (bias instanceof Float32Array && bias.length === d.N), 'qlinear_requant bias');
    need(typeof d.sNext === 'number', 'qlinear_requant needs the static scale sNext');
    const dxq = dev.get('xq', d.M * d.K), dsx = dev.get('sx', bytesOf(sx));
    const dwq = dev.get('wq', d.N * d.K), dws = dev.get('ws', 8 * d.N);
    const db = bias ? dev.get('bias', 4 * d.N) : null, dout = dev.get('out', d.M * d.N);
    A.upload(dxq, xq);
    A.upload(dsx, sx);
    A.upload(dwq, wq);
    A.upload(dws, ws);
    if (bias) A.upload(db, bias);
    A.gemmRequant(dxq, dwq, d.M, d.N, d.K, dsx, perTensor ? A.Q8_PER_TENSOR : A.Q8_PER_TOKEN,
                  dws, A.Q8_PER_CHANNEL, A.Q8_EPI_ROWCOL, 0, db, A[ACT_CODE[d.act || 'none']], d.sNext, dout);
    A.download(out, dout);
    return out;
  }
  if (d.op === 'qlinear_w4') {
    // decode linear with 4-bit per-group weights: x fp32 [M,K], per-token
    // int8 quantize, then the W4A8 GEMV; wq4 uint8 [N, K/2] (two codes per
    // byte), sw f64 [N * K / group]
    const x = args[d.xIdx], wq = args[d.wqIdx], sw = args[d.swIdx], out = args[d.outIdx];
    const bias = d.biasIdx === undefined || d.biasIdx < 0 ? null : args[d.biasIdx];
    need(x instanceof Float32Array && x.length === d.M * d.K, 'qlinear_w4 x');
    need(wq instanceof Uint8Array && wq.length === d.N * d.K / 2, 'qlinear_w4 packed weights');
    need(d.group > 0 && d.K % d.group === 0, 'qlinear_w4 group must divide K');
    need(sw instanceof Float64Array && sw.length === d.N * d.K / d.group, 'qlinear_w4 group scales');
    need(out instanceof Float32Array && out.length === d.M * d.N, 'qlinear_w4 out');
    need(bias === null || (bias instanceof Float32Array && bias.length === d.N), 'qlinear_w4 bias');
    const dx = dev.get('x', 4 * d.M * d.K), dxq = dev.get('xq', d.M * d.K), dsx = dev.get('sx', 8 * d.M);
    const dwq = dev.get('wq', bytesOf(wq)), dsw = dev.get('sw', bytesOf(sw));
    const db = bias ? dev.get('bias', 4 * d.N) : null, dout = dev.get('out', 4 * d.M * d.N);
    A.upload(dx, x);
    A.upload(dwq, wq);
    A.upload(dsw, sw);
    if (bias) A.upload(db, bias);
    A.quantizeRows(dx, d.M, d.K, A.Q8_PER_TOKEN, dxq, dsx);
    A.gemvW4(dxq, dsx, A.Q8_PER_TOKEN, dwq, dsw, d.M, d.N, d.K, d.group, db, A[ACT_CODE[d.act || 'none']], dout);
    A.download(out, dout);
    return out;
  }
  throw new Error(`hip backend: unknown op '${d.op}'`);
}

/** The object registerBackend('hip', ...) takes (backend_registry.ts:14-20). */
function createHipRuntimeBackend() {
  return {
    instantiate(kernel) {
      const d = kernel && kernel.metadata && kernel.metadata.q8;
      need(kernel && kernel.metadata && kernel.metadata.kind === HIP_KIND, 'kernel kind is not hip');
      need(d && typeof d.op === 'string', 'kernel metadata carries no q8 descriptor');
      return { kernel, desc: d, dev: new DeviceArgs() };
    },
    runSync(inst, tensorArgs, shapeValues) {
      need(shapeValues === null || shapeValues === undefined || shapeValues.length === 0,
           'dynamic shapes are not supported by the int8 kernels');
      return runDescriptor(inst.desc, tensorArgs, inst.dev);
    },
    runAsync(inst, tensorArgs, shapeValues) {
      return Promise.resolve().then(() => this.runSync(inst, tensorArgs, shapeValues));
    },
    isAsync() { return false; },
  };
}

/** registerExternalCodegen('hip_int8', ...) entry (codegen_registry.ts:17-21). */
function createHipExternalCodegen() {
  return {
    targetKind: HIP_KIND,
    runtimeKind: HIP_KIND,
    compile(primFunc, target, info) {
      return { source: '', metadata: { kind: HIP_KIND, q8: info, outputIndices: info.outputIndices } };
    },
  };
}

/** registerExternalCodegenProvider(...) entry (external_codegen.ts:11-17). */
function createHipProvider(EXTERNAL_CODEGEN_ATTR) {
  const attr = EXTERNAL_CODEGEN_ATTR || 'external_codegen';    // FuncAttr.EXTERNAL_CODEGEN
  return {
    name: PROVIDER,
    enabled(config, target) {
      const t = target && (target.kind || (target.features && target.features.kind));
      return t === HIP_KIND && !!(config && config.quantization && config.quantization.enabled);
    },
    annotate(tirModule) {
      for (const primFunc of tirModule) {
        const info = detectInt8Kernel(primFunc);
        if (info) primFunc.setAttr(attr, { name: PROVIDER, info });
      }
    },
  };
}

/** A compile target for the hip kind (support/target.ts: kind is a free string). */
function hipTarget() {
  return { kind: HIP_KIND, isGPU: () => true, supportsInt8: true };
}

// ---------------------------------------------------------------- eager library
/**
 * Registers the dynamic int8 ops with the dispatcher.  `tensors` adapts the
 * host's tensor type: { data(t) -> typed array, shape(t) -> number[],
 * make(typedArray, shape) -> tensor }.
 */
function defineEagerLibrary(Library, DispatchKey, tensors) {
  const lib = new Library('q8', 'DEF');
  const dev = new DeviceArgs();
  const rowsOf = (shape) => shape.slice(0, -1).reduce((a, b) => a * b, 1);
  lib.def('quantize_per_token(Tensor x) -> (Tensor, Tensor)')
    .impl('quantize_per_token', DispatchKey.GPU, (x) => {
      const data = tensors.data(x), shape = tensors.shape(x);
      const K = shape[shape.length - 1], M = rowsOf(shape);
      const A = q8();
      const dx = dev.get('x', 4 * M * K), dq = dev.get('q', M * K), ds = dev.get('s', 8 * M);
      A.upload(dx, data);
      A.quantizeRows(dx, M, K, A.Q8_PER_TOKEN, dq, ds);
      const q = new Int8Array(M * K), s = new Float64Array(M);
      A.download(q, dq);
      A.download(s, ds);
      return [tensors.make(q, shape), tensors.make(s, [M])];
    });
  lib.def('dequantize_per_token(Tensor q, Tensor scales) -> Tensor')
    .impl('dequantize_per_token', DispatchKey.GPU, (q, scales) => {
      const data = tensors.data(q), shape = tensors.shape(q), s = tensors.data(scales);
      const K = shape[shape.length - 1], M = rowsOf(shape);
      const A = q8();
      const dq = dev.get('q', M * K), ds = dev.get('s', 8 * M), dy = dev.get('y', 4 * M * K);
      A.upload(dq, data);
      A.upload(ds, s);
      A.dequantize(dq, A.Q8_I8, M, K, ds, A.Q8_PER_TOKEN, 0, dy);
      const y = new Float32Array(M * K);
      A.download(y, dy);
      return tensors.make(y, shape);
    });
  lib.def('qlinear(Tensor x, Tensor w_q, Tensor w_scales, Tensor bias) -> Tensor')
    .impl('qlinear', DispatchKey.GPU, (x, wq, ws, bias) => {
      const xs = tensors.shape(x), K = xs[xs.length - 1], M = rowsOf(xs);
      const N = tensors.shape(wq)[0];
      const out = new Float32Array(M * N);
      const args = [tensors.data(x), tensors.data(wq), tensors.data(ws), bias ? tensors.data(bias) : null, out];
      runDescriptor({ op: 'qlinear', M, N, K, xIdx: 0, wqIdx: 1, wsIdx: 2, biasIdx: bias ? 3 : -1,
                      outIdx: 4, granularity: 'per_token', act: 'none' }, args, dev);
      return tensors.make(out, xs.slice(0, -1).concat([N]));
    });
  return lib;
}

/**
 * Plugs the hip int8 path into a running mlfw.  `r` carries the reference's
 * registry functions: { registerBackend, registerExternalCodegen,
 * registerExternalCodegenProvider, FuncAttr?, Library?, DispatchKey?, tensors? }.
 */
function registerHip(r) {
  need(r && typeof r.registerBackend === 'function', 'registerBackend is required');
  r.registerBackend(HIP_KIND, createHipRuntimeBackend());
  if (r.registerExternalCodegen) r.registerExternalCodegen(PROVIDER, createHipExternalCodegen());
  if (r.registerExternalCodegenProvider) {
    r.registerExternalCodegenProvider(createHipProvider(r.FuncAttr && r.FuncAttr.EXTERNAL_CODEGEN));
  }
  let library = null;
  if (r.Library && r.DispatchKey && r.tensors) library = defineEagerLibrary(r.Library, r.DispatchKey, r.tensors);
  return { kind: HIP_KIND, provider: PROVIDER, library };
}

module.exports = {
  HIP_KIND, PROVIDER, registerHip, createHipRuntimeBackend, createHipExternalCodegen,
  createHipProvider, defineEagerLibrary, detectInt8Kernel, runDescriptor, hipTarget, DeviceArgs,
};
