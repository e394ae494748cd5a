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
// Target attribute (TargetFeatures.withAttr, support/target.ts:145-147) that
// selects how a compiled plan quantizes activations: 'static' (the
// calibrated scales of QuantizationPass, the reference's semantics),
// 'per_token' or 'per_tensor' (absmax scales taken at run time).
const ACTIVATIONS_ATTR = 'q8_activations';
const ACTIVATION_MODES = new Set(['static', 'per_token', 'per_tensor']);

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

// ---------------------------------------------------------------- device residency
// Constant tensors (a kernel's constant buffers: QuantizationPass's int8
// weights and f32 scale vectors, src/compiler/passes/lowering/graph_to_tensor.ts:
// 210-239) keep one device copy per host typed array, uploaded on first use
// -- the rule of the reference CUDA runtime's resident mirrors
// (src/runtime/node/cuda/resident.ts:129-140, cuda_runtime.ts:123-146).  A
// derived form (the [N,K] transpose of a [K,N] weight, f64 widening of an
// f32 scale vector) is cached beside it.  markHostDirty(array) drops the
// copies of an array the host rewrote.
const stats = { uploadBytes: 0, constUploadBytes: 0, downloadBytes: 0, launches: 0, fusedLinears: 0,
                dynamicLinears: 0, residentSkips: 0, graphCaptures: 0, graphReplays: 0 };
const _resident = new WeakMap();

function resetStats() { for (const k of Object.keys(stats)) stats[k] = 0; }

function upload(dbuf, host, isConst) {
  q8().upload(dbuf, host);
  stats.uploadBytes += host.byteLength;
  if (isConst) stats.constUploadBytes += host.byteLength;
}

function download(host, dbuf) {
  q8().download(host, dbuf);
  stats.downloadBytes += host.byteLength;
}

function residentConst(arr, variant, derive) {
  let m = _resident.get(arr);
  if (!m) { m = new Map(); _resident.set(arr, m); }
  let b = m.get(variant);
  if (!b) {
    const host = derive ? derive(arr) : arr;
    b = q8().alloc(Math.max(host.byteLength, 1));
    upload(b, host, true);
    m.set(variant, b);
  }
  if (_recordConsts) _recordConsts.push(b);
  return b;
}

/**
 * The tap-major device copy of a constant int8 conv weight (convWeightTaps,
 * made from its resident plain copy on the first use), or null for weights
 * the conv uses as given: ui8 operands or zero points (the direct kernel),
 * channels per group not a multiple of 16, one kernel position.
 */
function residentConvTaps(arr, d) {
  const kn = numel(d.wShape.slice(2));
  if ((d.xDtype || 'i8') !== 'i8' || (d.wDtype || 'i8') !== 'i8' || d.zpX || d.zpW) return null;
  if (d.wShape[1] % 16 !== 0 || kn < 2 || kn > 1024) return null;
  let m = _resident.get(arr);
  if (!m) { m = new Map(); _resident.set(arr, m); }
  let t = m.get('taps');
  if (!t) {
    const plain = residentConst(arr, 'plain');
    t = q8().alloc(Math.max(arr.byteLength, 1));
    q8().convWeightTaps(plain, d.d, d.wShape, d.groups, t);
    m.set('taps', t);
  }
  if (_recordConsts) _recordConsts.push(t);
  return t;
}

function markHostDirty(arr) {
  _resident.delete(arr);
  _constEpoch++;
}

// ---------------------------------------------------------------- runtime backend
const SRC_CODE = { i8: 'Q8_I8', ui8: 'Q8_U8', i32: 'Q8_I32' };
const ACT_CODE = { none: 'Q8_ACT_NONE', relu: 'Q8_ACT_RELU', silu: 'Q8_ACT_SILU' };

/** Device buffers of one kernel instance (or plan), reused across runs. */
class DeviceArgs {
  // graphed: the owner captures graphs that may name these buffers
  constructor(graphed = false) { this.bufs = new Map(); this.epoch = 0; this.retired = []; this.graphed = graphed; }
  get(key, bytes) {
    let b = this.bufs.get(key);
    if (!b || q8().bytes(b) < bytes) {
      // a replaced buffer may still be named by a captured graph: it is
      // retired, not freed, until the owner drops that graph
      if (b && this.graphed) this.retired.push(b);
      else if (b) q8().free(b);
      b = q8().alloc(Math.max(bytes, 1));
      this.bufs.set(key, b);
      this.epoch++;
    }
    return b;
  }
  f64(key, values) {                    // a small constant f64 array, uploaded once
    const k = `${key}:${values.join(',')}`;
    let b = this.bufs.get(k);
    if (!b) {
      b = q8().alloc(8 * values.length);
      upload(b, new Float64Array(values), true);
      this.bufs.set(k, b);
      this.epoch++;
    }
    return b;
  }
  live() { return [...this.bufs.values()]; }
  freeRetired() {
    for (const b of this.retired) q8().free(b);
    this.retired = [];
  }
  release() {
    for (const b of this.bufs.values()) q8().free(b);
    for (const b of this.retired) q8().free(b);
    this.bufs.clear();
    this.retired = [];
  }
}

function need(cond, msg) {
  if (!cond) throw new Error(`hip backend: ${msg}`);
}

function transposeI8(b, rows, cols) {
  const t = new b.constructor(rows * cols);
  for (let r = 0; r < rows; r++) for (let c = 0; c < cols; c++) t[c * rows + r] = b[r * cols + c];
  return t;
}

const CTOR = { i8: Int8Array, ui8: Uint8Array, i32: Int32Array, f32: Float32Array, f64: Float64Array };
const ELEM_BYTES = { i8: 1, ui8: 1, i32: 4, f32: 4, f64: 8 };
const EW_DT = ['i8', 'ui8', 'i32', 'f32', 'f64'];          // Q8_I8 .. Q8_F64

/** Which tensor arguments a descriptor reads ({index: {ctor, n, what}}). */
function inputSpecs(d) {
  const s = new Map();
  const add = (i, ctor, n, what) => { if (i !== undefined && i >= 0) s.set(i, { ctor, n, what: `${d.op} ${what}` }); };
  switch (d.op) {
    case 'quantize': add(d.inIdx, Float32Array, d.n, 'input'); break;
    case 'dequantize': add(d.inIdx, CTOR[d.srcDtype], d.n, 'input'); break;
    case 'quantized_dot':
      add(d.aIdx, CTOR[d.aDtype || 'i8'], d.M * d.K, 'lhs');
      add(d.bIdx, CTOR[d.bDtype || 'i8'], d.N * d.K, 'rhs');
      break;
    case 'quantized_conv':
      add(d.xIdx, CTOR[d.xDtype || 'i8'], numel(d.xShape), 'input');
      add(d.wIdx, CTOR[d.wDtype || 'i8'], numel(d.wShape), 'kernel');
      break;
    case 'qlinear':
      add(d.xIdx, Float32Array, d.M * d.K, 'x'); add(d.wqIdx, Int8Array, d.N * d.K, 'wq');
      add(d.wsIdx, Float64Array, d.N, 'weight scales'); add(d.biasIdx, Float32Array, d.N, 'bias');
      break;
    case 'qlinear_requant':
      need(typeof d.sNext === 'number', 'qlinear_requant needs the static scale sNext');
      add(d.xqIdx, Int8Array, d.M * d.K, 'xq');
      add(d.sxIdx, Float64Array, d.granularity === 'per_tensor' ? 1 : d.M, 'activation scales');
      add(d.wqIdx, Int8Array, d.N * d.K, 'wq'); add(d.wsIdx, Float64Array, d.N, 'weight scales');
      add(d.biasIdx, Float32Array, d.N, 'bias');
      break;
    case 'qlinear_w4':
      need(d.group > 0 && d.K % d.group === 0, 'qlinear_w4 group must divide K');
      add(d.xIdx, Float32Array, d.M * d.K, 'x'); add(d.wqIdx, Uint8Array, d.N * d.K / 2, 'packed weights');
      add(d.swIdx, Float64Array, d.N * d.K / d.group, 'group scales'); add(d.biasIdx, Float32Array, d.N, 'bias');
      break;
    case 'ewise':
      d.inputIdx.forEach((p, j) => {
        if (!s.has(p)) s.set(p, { ctor: CTOR[EW_DT[d.prog.inDtype[j]]], n: d.inNumel[j], min: true, what: `ewise input ${j}` });
      });
      break;
    default: throw new Error(`hip backend: unknown op '${d.op}'`);
  }
  return s;
}

/** Output arguments of a descriptor ({index: {ctor, n, what}}). */
function outputSpecs(d) {
  const s = new Map();
  const set = (ctor, n) => s.set(d.outIdx, { ctor, n, what: `${d.op} out` });
  switch (d.op) {
    case 'quantize': set(d.targetDtype === 'ui8' ? Uint8Array : Int8Array, d.n); break;
    case 'dequantize': set(Float32Array, d.n); break;
    case 'quantized_dot': set(Int32Array, d.M * d.N); break;
    case 'quantized_conv': set(Int32Array, numel(d.outShape)); break;
    case 'qlinear': case 'qlinear_w4': set(Float32Array, d.M * d.N); break;
    case 'qlinear_requant': set(Int8Array, d.M * d.N); break;
    case 'ewise': set(CTOR[EW_DT[d.prog.outDtype]], d.outNumel); break;
    default: throw new Error(`hip backend: unknown op '${d.op}'`);
  }
  return s;
}

function checkArg(a, spec) {
  need(a instanceof spec.ctor, `${spec.what} must be a ${spec.ctor.name}`);
  need(spec.min ? a.length >= spec.n : a.length === spec.n,
       `${spec.what} has ${a.length} elements, expected ${spec.n}`);
}

/**
 * Runs a descriptor on device buffers: `dv[i]` is the device buffer of
 * tensor argument i; `rhsNK` (quantized_dot) is the weight already in the
 * [N,K] layout when the caller has it.
 */
function execDevice(d, dv, dev, rhsNK, wTaps) {
  const A = q8();
  stats.launches++;
  switch (d.op) {
    case 'quantize':
      A.quantizeStatic(dv[d.inIdx], d.n, d.scale, d.zeroPoint, A[d.targetDtype === 'ui8' ? 'Q8_U8' : 'Q8_I8'], dv[d.outIdx]);
      return;
    case 'dequantize':
      A.dequantize(dv[d.inIdx], A[SRC_CODE[d.srcDtype]], 1, d.n, dev.f64('s', [d.scale]), A.Q8_PER_TENSOR,
                   d.zeroPoint, dv[d.outIdx]);
      return;
    case 'quantized_dot': {
      const aD = (d.aDtype || 'i8') === 'ui8' ? A.Q8_U8 : A.Q8_I8, bD = (d.bDtype || 'i8') === 'ui8' ? A.Q8_U8 : A.Q8_I8;
      let b = rhsNK;
      if (!b) {
        b = dv[d.bIdx];
        if (d.rhsLayout === 'KN') {        // [K,N] -> [N,K] on the device
          const t = dev.get('bT', d.N * d.K);
          A.ewise(transposeProg(d.K, d.N, bD === A.Q8_U8 ? 1 : 0), [b], [d.N * d.K], t, d.N * d.K);
          b = t;
        }
      }
      const ws = A.quantizedDotWorkspace(d.M, d.N, d.K, aD, bD, d.zpA, d.zpB);
      A.quantizedDot(dv[d.aIdx], aD, b, bD, d.M, d.N, d.K, d.zpA, d.zpB, ws > 0 ? dev.get('ws', ws) : null,
                     dv[d.outIdx]);
      return;
    }
    case 'quantized_conv': {
      const xD = (d.xDtype || 'i8') === 'ui8' ? A.Q8_U8 : A.Q8_I8, wD = (d.wDtype || 'i8') === 'ui8' ? A.Q8_U8 : A.Q8_I8;
      const ws = A.convWorkspace(d.d, d.xShape, d.wShape, d.strides, d.padLo, d.padHi, d.dilation, d.groups);
      if (wTaps) {            // a constant weight, prepacked once
        A.quantizedConvPrepacked(dv[d.xIdx], dv[d.wIdx], wTaps, d.d, d.xShape, d.wShape, d.strides, d.padLo, d.padHi,
                                 d.dilation, d.groups, d.zpX, d.zpW, A.Q8_I32, 0, ws > 0 ? dev.get('ws', ws) : null,
                                 dv[d.outIdx]);
        return;
      }
      A.quantizedConvEx(dv[d.xIdx], xD, dv[d.wIdx], wD, d.d, d.xShape, d.wShape, d.strides, d.padLo, d.padHi,
                        d.dilation, d.groups, d.zpX, d.zpW, A.Q8_I32, 0, ws > 0 ? dev.get('ws', ws) : null,
                        dv[d.outIdx]);
      return;
    }
    case 'qlinear': {
      // dynamic per-token int8 linear: x fp32 [M,K]; wq int8 [N,K] + f64 scales [N];
      // quantize + GEMM + epilogue in one call (one kernel for a single token)
      const perTensor = d.granularity === 'per_tensor';
      A.qlinearDynamic(dv[d.xIdx], d.M, d.K, perTensor ? A.Q8_PER_TENSOR : A.Q8_PER_TOKEN, dv[d.wqIdx], dv[d.wsIdx],
                       A.Q8_PER_CHANNEL, d.N, d.biasIdx >= 0 ? dv[d.biasIdx] : null, A[ACT_CODE[d.act || 'none']],
                       dv[d.outIdx], dev.get('xq', d.M * d.K), dev.get('sx', 8 * (perTensor ? 1 : d.M)));
      return;
    }
    case 'qlinear_requant': {
      // int8 codes in, the next layer's static-scale codes out (the calibrated
      // chain ... mul(sv) -> add(b) -> max -> quantize)
      const perTensor = d.granularity === 'per_tensor';
      A.gemmRequant(dv[d.xqIdx], dv[d.wqIdx], d.M, d.N, d.K, dv[d.sxIdx], perTensor ? A.Q8_PER_TENSOR : A.Q8_PER_TOKEN,
                    dv[d.wsIdx], A.Q8_PER_CHANNEL, A.Q8_EPI_ROWCOL, 0, d.biasIdx >= 0 ? dv[d.biasIdx] : null,
                    A[ACT_CODE[d.act || 'none']], d.sNext, dv[d.outIdx]);
      return;
    }
    case 'qlinear_w4': {
      // decode linear with 4-bit per-group weights: per-token int8 quantize of
      // x, then the W4A8 GEMV
      const dxq = dev.get('xq', d.M * d.K), dsx = dev.get('sx', 8 * d.M);
      A.quantizeRows(dv[d.xIdx], d.M, d.K, A.Q8_PER_TOKEN, dxq, dsx);
      A.gemvW4(dxq, dsx, A.Q8_PER_TOKEN, dv[d.wqIdx], dv[d.swIdx], d.M, d.N, d.K, d.group,
               d.biasIdx >= 0 ? dv[d.biasIdx] : null, A[ACT_CODE[d.act || 'none']], dv[d.outIdx]);
      return;
    }
    case 'ewise':
      A.ewise(d.progBytes || (d.progBytes = ew().packProg(d.prog)), d.inputIdx.map((p) => dv[p]), d.inNumel,
              dv[d.outIdx], d.outNumel);
      return;
    default:
      throw new Error(`hip backend: unknown op '${d.op}'`);
  }
}

// [N,K] <- [K,N] gather as an elementwise program (out[n,k] = in[k,n])
const _tpCache = new Map();
function transposeProg(K, N, unsigned) {
  const key = `${K}x${N}:${unsigned}`;
  let p = _tpCache.get(key);
  if (!p) {
    const dt = unsigned ? 1 : 0;
    const coef = [1, N, 0, 0, 0, 0, 0];
    p = ew().packProg({ ndims: 2, ninputs: 1, extent: [N, K], inDtype: [dt], inCoef: [coef], outDtype: dt,
                        ncode: 1, result: 0, nconst: 0, code: [{ op: ew().OP.LOAD, dst: 0, a: 0, b: 0, c: 0, aux: 0, rnd: 0 }],
                        konst: [] });
    _tpCache.set(key, p);
  }
  return p;
}

function ew() { return require('./ewise.js'); }

/**
 * Runs one descriptor on host typed arrays: inputs are uploaded (constant
 * buffers only once, see residentConst), the op runs on the device, the
 * outputs are downloaded into the caller's arrays (the outputIndices rule of
 * the reference CUDA runtime, cuda_runtime.ts:85-121).
 */
function runDescriptor(d, args, dev, consts) {
  const ins = inputSpecs(d), outs = outputSpecs(d);
  // every argument is checked before the first device call
  for (const [i, spec] of ins) checkArg(args[i], spec);
  for (const [i, spec] of outs) checkArg(args[i], spec);
  const dv = [];
  let rhsNK = null;
  for (const [i] of ins) {
    const a = args[i];
    const isConst = !!(consts && consts.has(a));
    if (d.op === 'quantized_dot' && i === d.bIdx && d.rhsLayout === 'KN') {
      rhsNK = isConst ? residentConst(a, 'T', (w) => transposeI8(w, d.K, d.N)) : null;
      if (!rhsNK) {
        rhsNK = dev.get('bT', d.N * d.K);
        upload(rhsNK, transposeI8(a, d.K, d.N), false);
      }
      continue;
    }
    if (isConst) { dv[i] = residentConst(a, 'plain'); continue; }
    dv[i] = dev.get(`in${i}`, a.byteLength);
    upload(dv[i], a, false);
  }
  for (const [i] of outs) dv[i] = dev.get(`out${i}`, args[i].byteLength);
  const wTaps = d.op === 'quantized_conv' && consts && consts.has(args[d.wIdx]) ? residentConvTaps(args[d.wIdx], d) : null;
  execDevice(d, dv, dev, rhsNK, wTaps);
  for (const [i] of outs) download(args[i], dv[i]);
  return args[d.outIdx];
}

/** Constant-buffer arrays of a compiled kernel (metadata.constBuffers). */
function constSet(kernel) {
  const s = new Set();
  const cbs = kernel && kernel.metadata && kernel.metadata.constBuffers;
  if (cbs) for (const cb of cbs) if (cb && cb.data) s.add(cb.data);
  return s;
}

// ---------------------------------------------------------------- plan execution
/**
 * runPlan (backend_registry.ts:14-20, RuntimeModule.runPlanAsync,
 * runtime.ts:290-329), the hip form of the reference's CUDA plan runner
 * (src/runtime/node/cuda/device_plan.ts:178-297): every step is a hip
 * kernel, so the whole plan runs with its slots on the device.
 *  - Every step's arguments (plan slots and the kernel's constant buffers)
 *    are checked against its descriptor before anything is uploaded or
 *    launched, as runSync checks them.
 *  - Slots share device memory by the plan's buffer assignment
 *    (plan.buffers.slotBuffer / bufferBytes, the compiler's lifetime-based
 *    groups, _groupsOf in device_plan.ts:44-60); without one every slot has
 *    its own buffer.  Buffers stay with the plan across calls.
 *  - Plan inputs (slots read before any step writes them) are uploaded;
 *    with opts.resident (tracing/compile.ts:115) an input whose
 *    RuntimeTensor.resident {key, version} (runtime.ts:128) is what the last
 *    call uploaded into the same buffer is not uploaded again
 *    (device_plan.ts:220-262).  Intermediates never leave the device, and
 *    only the slots the caller reads back are downloaded.
 *  - A quantized_dot whose int32 result feeds only the per-channel epilogue
 *    group of the next step (matchEpilogue: convert -> mul(sv) [-> add(b)]
 *    [-> max(0)] [-> quantize]) runs as one fused GEMM launch (q8_gemm /
 *    q8_gemm_requant), and the int32 tensor is never written.
 *  - With HIP graphs on (setHipGraphEnabled, the reference's
 *    setCudaGraphEnabled; or opts.graph), the first call runs eagerly, the
 *    second captures the plan's launches on the addon's stream and every
 *    later call replays the graph (device_plan.ts:178-218).  The graph is
 *    dropped and re-captured when a buffer it names changes (a slot group
 *    grows, a constant buffer is marked dirty).
 *  - runPlan enqueues the plan's uploads and launches on the addon's stream
 *    and returns; its promise settles once the device has finished
 *    (syncAsync: the wait runs on a worker thread, so the JS thread is free
 *    meanwhile) and the outputs are downloaded.  The reference's CUDA
 *    runner blocks the JS thread for the whole plan instead (devSync in
 *    device_plan.ts:254,276 inside the async runCudaPlan, :288-299).  All
 *    plans share one stream, and a plan's downloads must read its own
 *    results, so an asynchronous run waits for the previous one to settle
 *    before it uploads anything; runPlanSync and releasePlan throw while
 *    an asynchronous run of the plan is in flight.
 */
const _planState = new WeakMap();
let _planTail = null;        // the last asynchronous plan run, settled or not; null when none is in flight
let _useHipGraph = false;
/** The reference's setCudaGraphEnabled / isCudaGraphEnabled (device_plan.ts:40-42). */
function setHipGraphEnabled(on) { _useHipGraph = !!on; }
function isHipGraphEnabled() { return _useHipGraph; }

function slotBytes(t) { return t && t.data ? t.data.byteLength : 0; }

/** Slot -> buffer group (device_plan.ts _groupsOf). */
function groupsOf(plan) {
  const b = plan.buffers;
  const count = b ? b.bufferBytes.length : plan.numSlots;
  const of = new Array(plan.numSlots);
  for (let s = 0; s < plan.numSlots; s++) of[s] = b ? b.slotBuffer[s] : s;
  return { of, count };
}

function planStateOf(plan) {
  let st = _planState.get(plan);
  if (!st) {
    st = { dev: new DeviceArgs(true), inst: new Map(), gbuf: [], pin: new Map(), graph: null, graphKeep: null,
           warm: false, noGraph: false, epoch: -1, devEpoch: -1 };
    _planState.set(plan, st);
  }
  return st;
}

/** Frees a plan's device buffers and graph (releaseAllPlanBuffers for one plan). */
function releasePlan(plan) {
  const st = _planState.get(plan);
  if (!st) return;
  need(!st.inFlight, 'releasePlan: an asynchronous runPlan of this plan is still in flight; await it first');
  dropGraph(st);
  for (const b of st.gbuf) if (b) q8().free(b);
  st.dev.release();
  _planState.delete(plan);
}

function dropGraph(st) {
  if (st.graph) q8().graphDestroy(st.graph);
  st.graph = null;
  st.graphKeep = null;
  st.warm = false;
  st.dev.freeRetired();
}

// constant buffers marked dirty since a graph was captured invalidate it
let _constEpoch = 0;
let _recordConsts = null;

function checkStepArgs(s, inst, slots) {
  const d = inst.desc;
  const io = s.inputSlots.concat(s.outputSlots);
  const argAt = (i) => (i < io.length ? (slots[io[i]] ? slots[io[i]].data : undefined) : inst.constData[i - io.length]);
  for (const [i, spec] of inputSpecs(d)) checkArg(argAt(i), spec);
  for (const [i, spec] of outputSpecs(d)) checkArg(argAt(i), spec);
}

function runPlanOnDevice(plan, slots, steps, opts) {
  need(!(_planState.get(plan) || {}).inFlight,
       'runPlanSync: an asynchronous runPlan of this plan is still in flight; await it first');
  const finish = enqueuePlan(plan, slots, steps, opts);
  q8().sync();
  finish();
}

/** runPlan's promise form: the plan's work is enqueued when no earlier
 * asynchronous run is in flight, else when that run settles. */
function runPlanAsync(plan, slots, steps, opts) {
  const start = () => {
    const st = planStateOf(plan);
    need(!st.inFlight, 'runPlan: the plan is still in flight');
    const finish = enqueuePlan(plan, slots, steps, opts);
    st.inFlight = true;
    return q8().syncAsync().then(() => { st.inFlight = false; finish(); },
                                 (e) => { st.inFlight = false; throw e; });
  };
  let p;
  if (_planTail === null) {
    try { p = start(); } catch (e) { return Promise.reject(e); }
  } else {
    p = _planTail.then(start);
  }
  const tail = p.then(() => {}, () => {});
  _planTail = tail;
  tail.then(() => { if (_planTail === tail) _planTail = null; });
  return p;
}

/** Checks, uploads and launches a plan on the addon's stream; returns the
 * function that downloads its outputs once the stream has finished. */
function enqueuePlan(plan, slots, steps, opts) {
  const st = planStateOf(plan);
  const dev = st.dev;
  const instOf = (kernel) => {
    let i = st.inst.get(kernel);
    if (!i) {
      const d = kernel && kernel.metadata && kernel.metadata.q8;
      need(kernel && kernel.metadata && kernel.metadata.kind === HIP_KIND && d, `plan step is not a hip kernel`);
      i = { desc: d, consts: constSet(kernel), constData: (kernel.metadata.constBuffers || []).map((c) => c.data) };
      st.inst.set(kernel, i);
    }
    return i;
  };
  // every argument of every step is checked before the first device call
  steps.forEach((s) => {
    need(!s.shapeValues || s.shapeValues.length === 0, 'dynamic shapes are not supported by the int8 kernels');
    checkStepArgs(s, instOf(s.kernel), slots);
  });
  const produced = new Map(), readers = new Map();
  steps.forEach((s, k) => {
    for (const o of s.outputSlots) if (!produced.has(o)) produced.set(o, k);
    for (const i of s.inputSlots) { if (!readers.has(i)) readers.set(i, []); readers.get(i).push(k); }
  });
  const argSet = new Set(plan.argSlots);
  const hostNeeds = new Set();
  for (const a of plan.argSlots) if (produced.has(a)) hostNeeds.add(a);
  for (const fx of plan.returnFixups || []) if (fx.kind === 'copy') hostNeeds.add(fx.srcSlot);

  // device memory: one buffer per slot group, sized for its largest slot
  const groups = groupsOf(plan);
  const wanted = new Array(groups.count).fill(0);
  const members = new Array(groups.count).fill(0);
  for (let s = 0; s < plan.numSlots; s++) {
    if (!slots[s] || !slots[s].data) continue;
    const g = groups.of[s];
    wanted[g] = Math.max(wanted[g], slotBytes(slots[s]), 1);
    members[g]++;
  }
  for (let g = 0; g < groups.count; g++) {
    if (!wanted[g] || (st.gbuf[g] && q8().bytes(st.gbuf[g]) >= wanted[g])) continue;
    dropGraph(st);                                   // the graph names the old buffer
    if (st.gbuf[g]) q8().free(st.gbuf[g]);
    st.gbuf[g] = q8().alloc(wanted[g]);
    for (let s = 0; s < plan.numSlots; s++) if (groups.of[s] === g) st.pin.delete(s);
  }
  const slotBuf = (s) => {
    const b = st.gbuf[groups.of[s]];
    need(b, `plan slot ${s} has no device buffer`);
    return b;
  };

  // plan inputs: slots read before any step writes them (resident pins
  // only for slots alone in their buffer, which no step overwrites)
  const resident = !!(opts && opts.resident);
  for (let s = 0; s < plan.numSlots; s++) {
    const t = slots[s];
    if (!t || !t.data) continue;
    const first = produced.has(s) ? produced.get(s) : Infinity;
    const rd = readers.get(s) || [];
    if (!rd.some((k) => k <= first)) continue;
    const res = t.resident;
    if (resident && res && first === Infinity && members[groups.of[s]] === 1) {
      const prev = st.pin.get(s);
      if (prev && prev.key === res.key && prev.version === res.version && prev.data === t.data) {
        stats.residentSkips++;
        continue;
      }
      st.pin.set(s, { key: res.key, version: res.version, data: t.data });
    } else {
      st.pin.delete(s);
    }
    upload(slotBuf(s), t.data, false);
  }

  const devArgs = (s, inst) => {
    const dv = [];
    const all = s.inputSlots.concat(s.outputSlots);
    all.forEach((slot, i) => { dv[i] = slotBuf(slot); });
    inst.constData.forEach((data, j) => { dv[all.length + j] = residentConst(data, 'plain'); });
    return dv;
  };
  const hostArgs = (s, inst) => s.inputSlots.concat(s.outputSlots).map((slot) => slots[slot] && slots[slot].data)
    .concat(inst.constData);
  const launchAll = () => {
    for (let k = 0; k < steps.length; k++) {
      const s = steps[k], inst = instOf(s.kernel), d = inst.desc;
      const mode = (opts && opts.q8Activations) || d.activations || 'static';
      if (d.op === 'quantize' && mode !== 'static' && k + 2 < steps.length) {
        need(ACTIVATION_MODES.has(mode), `unknown q8 activation mode '${mode}'`);
        if (tryDynamicLinear(mode, s, d, steps[k + 1], instOf(steps[k + 1].kernel), steps[k + 2],
                             instOf(steps[k + 2].kernel), slots, readers, argSet, hostNeeds, slotBuf, dev, hostArgs)) {
          k += 2;
          continue;
        }
      }
      const fused = !(opts && opts.fuse === false) && k + 1 < steps.length &&
                    tryFusedLinear(s, inst, steps[k + 1], instOf(steps[k + 1].kernel), slots, readers, argSet,
                                   hostNeeds, slotBuf, dev, hostArgs);
      if (fused) { k++; continue; }
      const dv = devArgs(s, inst);
      let rhsNK = null;
      if (d.op === 'quantized_dot' && d.rhsLayout === 'KN') {
        const b = hostArgs(s, inst)[d.bIdx];
        if (inst.consts.has(b)) rhsNK = residentConst(b, 'T', (w) => transposeI8(w, d.K, d.N));
      }
      let wTaps = null;
      if (d.op === 'quantized_conv') {
        const w = hostArgs(s, inst)[d.wIdx];
        if (inst.consts.has(w)) wTaps = residentConvTaps(w, d);
      }
      execDevice(d, dv, dev, rhsNK, wTaps);
    }
  };

  const graphOn = opts && opts.graph !== undefined ? !!opts.graph : _useHipGraph;
  if (st.graph && (st.epoch !== _constEpoch || st.devEpoch !== dev.epoch)) dropGraph(st);
  if (!graphOn || st.noGraph) {
    launchAll();
  } else if (st.graph) {
    q8().graphLaunch(st.graph);
    stats.graphReplays++;
  } else if (!st.warm) {
    launchAll();                     // fills every cache the launches read, so a capture allocates nothing
    st.warm = true;
  } else {
    const A = q8();
    const keep = [];
    A.captureBegin();
    _recordConsts = keep;
    let g = null;
    try {
      launchAll();
    } catch (e) {
      _recordConsts = null;
      try { A.graphDestroy(A.captureEnd()); } catch (e2) { /* the capture is void either way */ }
      st.noGraph = true;             // this plan runs eagerly from now on
      throw e;
    }
    _recordConsts = null;
    g = A.captureEnd();
    st.graph = g;
    st.graphKeep = keep.concat(st.dev.live());      // every buffer the graph names stays alive with it
    st.epoch = _constEpoch;
    st.devEpoch = dev.epoch;
    stats.graphCaptures++;
    A.graphLaunch(g);
    stats.graphReplays++;
  }
  return () => {
    for (const s of hostNeeds) if (slots[s] && slots[s].data) download(slots[s].data, slotBuf(s));
  };
}

/**
 * The per-token (or per-tensor) dynamic form of one linear, for plans
 * compiled with q8 activations 'per_token' / 'per_tensor' (hipTarget's
 * q8opts): QuantizationPass's quantize(x, s) -> quantized_dot(xq, W) ->
 * convert * sv[n] (+ bias) (-> max 0) chain (quantization_pass.ts:390-459)
 * runs as one q8_qlinear_dynamic call that quantizes x at run time instead
 * of with the calibrated static scale s.  The weight's own scale is not in
 * the plan, only sv[n] = fround(s * sW[n]); the call uses sv[n] / s (f64),
 * so y = fround(acc * fround(sx[m] * (sv[n] / s))) -- the static result
 * exactly when the dynamic scale equals s.  No counterpart in the reference
 * (its activation scales are static); chains whose epilogue requantizes
 * (max -> quantize fused) stay static.
 */
function tryDynamicLinear(mode, sq, dq, s0, i0, s1, i1, slots, readers, argSet, hostNeeds, slotBuf, dev, hostArgs) {
  const d0 = i0.desc, e = i1.desc;
  if (dq.targetDtype !== 'i8' || dq.zeroPoint !== 0 || !(dq.scale > 0)) return false;
  if (d0.op !== 'quantized_dot' || e.op !== 'ewise' || !e.epilogue || e.epilogue.quant) return false;
  if ((d0.aDtype || 'i8') !== 'i8' || (d0.bDtype || 'i8') !== 'i8' || d0.zpA || d0.zpB) return false;
  const xSlot = sq.inputSlots[dq.inIdx], xqSlot = sq.outputSlots[dq.outIdx - sq.inputSlots.length];
  if (d0.aIdx >= s0.inputSlots.length || s0.inputSlots[d0.aIdx] !== xqSlot) return false;
  if ((readers.get(xqSlot) || []).length !== 1 || argSet.has(xqSlot) || hostNeeds.has(xqSlot)) return false;
  const accSlot = s0.outputSlots[d0.outIdx - s0.inputSlots.length];
  const ep = e.epilogue;
  const args1 = s1.inputSlots.concat(s1.outputSlots);
  if (args1[ep.accParam] !== accSlot || ep.M !== d0.M || ep.N !== d0.N || d0.M * d0.K !== dq.n) return false;
  if ((readers.get(accSlot) || []).length !== 1 || argSet.has(accSlot) || hostNeeds.has(accSlot)) return false;
  const h1 = hostArgs(s1, i1);
  const sv = h1[ep.svParam];
  if (!(sv instanceof Float32Array) || !i1.consts.has(sv) || sv.length !== d0.N) return false;
  const bHost = hostArgs(s0, i0)[d0.bIdx];
  if (!i0.consts.has(bHost)) return false;
  const A = q8();
  const wq = d0.rhsLayout === 'KN' ? residentConst(bHost, 'T', (w) => transposeI8(w, d0.K, d0.N))
                                   : residentConst(bHost, 'plain');
  const s = dq.scale;
  const wEff = residentConst(sv, `dyn:${s}`, (x) => Float64Array.from(x, (v) => v / s));
  let bias = null;
  if (ep.biasParam >= 0) {
    const bh = h1[ep.biasParam];
    if (!(bh instanceof Float32Array) || bh.length !== d0.N) return false;
    bias = i1.consts.has(bh) ? residentConst(bh, 'plain') : (ep.biasParam < s1.inputSlots.length ? slotBuf(s1.inputSlots[ep.biasParam]) : null);
    if (!bias) return false;
  }
  const perTensor = mode === 'per_tensor';
  stats.launches++;
  stats.dynamicLinears++;
  A.qlinearDynamic(slotBuf(xSlot), d0.M, d0.K, perTensor ? A.Q8_PER_TENSOR : A.Q8_PER_TOKEN, wq, wEff, A.Q8_PER_CHANNEL,
                   d0.N, bias, ep.relu ? A.Q8_ACT_RELU : A.Q8_ACT_NONE, slotBuf(args1[e.outIdx]),
                   dev.get('dyn_xq', d0.M * d0.K), dev.get('dyn_sx', 8 * (perTensor ? 1 : d0.M)));
  return true;
}

function tryFusedLinear(s0, i0, s1, i1, slots, readers, argSet, hostNeeds, slotBuf, dev, hostArgs) {
  const d0 = i0.desc, e = i1.desc;
  if (d0.op !== 'quantized_dot' || e.op !== 'ewise' || !e.epilogue) return false;
  if ((d0.aDtype || 'i8') !== 'i8' || (d0.bDtype || 'i8') !== 'i8' || d0.zpA || d0.zpB) return false;
  const accSlot = s0.outputSlots[d0.outIdx - s0.inputSlots.length];
  const ep = e.epilogue;
  const args1 = s1.inputSlots.concat(s1.outputSlots);
  if (args1[ep.accParam] !== accSlot || ep.M !== d0.M || ep.N !== d0.N) return false;
  if ((readers.get(accSlot) || []).length !== 1 || argSet.has(accSlot) || hostNeeds.has(accSlot)) return false;
  const h1 = hostArgs(s1, i1);
  const sv = h1[ep.svParam];
  if (!(sv instanceof Float32Array) || !i1.consts.has(sv) || sv.length !== d0.N) return false;
  const A = q8();
  const h0 = hostArgs(s0, i0);
  const a = slotBuf(s0.inputSlots[d0.aIdx]);
  const bHost = h0[d0.bIdx];
  let b;
  if (i0.consts.has(bHost)) {
    b = d0.rhsLayout === 'KN' ? residentConst(bHost, 'T', (w) => transposeI8(w, d0.K, d0.N)) : residentConst(bHost, 'plain');
  } else {
    b = d0.bIdx < s0.inputSlots.length ? slotBuf(s0.inputSlots[d0.bIdx]) : null;
    if (!b || d0.rhsLayout === 'KN') return false;
  }
  // E-pc as q8_gemm's row x column epilogue: fround(acc * fround(1 * sv[n]))
  const sB = residentConst(sv, 'f64', (x) => Float64Array.from(x));
  const sA = dev.f64('one', [1]);
  let bias = null;
  if (ep.biasParam >= 0) {
    const bh = h1[ep.biasParam];
    if (!(bh instanceof Float32Array) || bh.length !== d0.N) return false;
    bias = i1.consts.has(bh) ? residentConst(bh, 'plain') : (ep.biasParam < s1.inputSlots.length ? slotBuf(s1.inputSlots[ep.biasParam]) : null);
    if (!bias) return false;
  }
  const out = slotBuf(args1[e.outIdx]);
  const act = ep.relu ? A.Q8_ACT_RELU : A.Q8_ACT_NONE;
  stats.launches++;
  stats.fusedLinears++;
  if (ep.quant) {
    A.gemmRequant(a, b, d0.M, d0.N, d0.K, sA, A.Q8_PER_TENSOR, sB, A.Q8_PER_CHANNEL, A.Q8_EPI_ROWCOL, 0, bias, act,
                  ep.quant.scale, out);
  } else {
    A.gemm(a, b, d0.M, d0.N, d0.K, 0, 0, sA, A.Q8_PER_TENSOR, sB, A.Q8_PER_CHANNEL, A.Q8_EPI_ROWCOL, 0, bias, act,
           A.Q8_F32, out);
  }
  return true;
}

/** The object registerBackend('hip', ...) takes (backend_registry.ts:14-20). */
function createHipRuntimeBackend() {
  return {
    instantiate(kernel) {
      const d = kernel && kernel.metadata && kernel.metadata.q8;
      need(kernel && kernel.metadata && kernel.metadata.kind === HIP_KIND, 'kernel kind is not hip');
      need(d && typeof d.op === 'string', 'kernel metadata carries no q8 descriptor');
      inputSpecs(d);                     // rejects unknown ops before any device call
      return { kernel, desc: d, dev: new DeviceArgs(), consts: constSet(kernel) };
    },
    runSync(inst, tensorArgs, shapeValues) {
      need(shapeValues === null || shapeValues === undefined || shapeValues.length === 0,
           'dynamic shapes are not supported by the int8 kernels');
      return runDescriptor(inst.desc, tensorArgs, inst.dev, inst.consts);
    },
    runAsync(inst, tensorArgs, shapeValues) {
      return Promise.resolve().then(() => this.runSync(inst, tensorArgs, shapeValues));
    },
    // enqueues the plan and settles when its outputs are downloaded
    // (runPlanAsync); argument errors reject the promise
    runPlan(plan, slots, steps, opts) {
      return runPlanAsync(plan, slots, steps, opts);
    },
    isAsync() { return false; },
  };
}

/** registerExternalCodegen('hip_int8', ...) entry (codegen_registry.ts:17-21).
 * The kernel's constant buffers travel in metadata.constBuffers, as
 * BackendPipeline.compile attaches them for the non-external path
 * (backend/pipeline.ts:49-55), so RuntimeModule appends them to the
 * kernel's arguments (runtime.ts:76-81, 246-258). */
function createHipExternalCodegen(CONST_BUFFERS_ATTR) {
  const cattr = CONST_BUFFERS_ATTR || 'const_buffers';
  return {
    targetKind: HIP_KIND,
    runtimeKind: HIP_KIND,
    compile(primFunc, target, info) {
      const mode = activationMode(target);
      if (mode !== 'static' && info && info.op === 'quantize') info = Object.assign({}, info, { activations: mode });
      const metadata = { kind: HIP_KIND, q8: info, outputIndices: info.outputIndices };
      const cbs = primFunc && typeof primFunc.getAttr === 'function' ? primFunc.getAttr(cattr) : null;
      if (cbs && cbs.length > 0) {
        metadata.constBuffers = cbs.map((cb) => ({ name: cb.buffer.name, dtype: cb.buffer.dtype, data: cb.data }));
      }
      return { source: '', metadata };
    },
  };
}

/** Descriptor of a PrimFunc for the hip provider: an int8 op of the path,
 * or an elementwise loop nest (q8_ewise), or null. */
function describe(primFunc, constBuffers) {
  const info = detectInt8Kernel(primFunc);
  if (info) return info;
  const tr = ew().translateEwise(primFunc);
  if (!tr) return null;
  const zeroData = new Map();
  for (const cb of constBuffers || []) {
    const data = cb.data;
    let allZero = data && data.length > 0;
    for (let i = 0; allZero && i < data.length; i++) allZero = Object.is(+data[i], 0);
    zeroData.set(cb.buffer.name, allZero);
  }
  const params = [];
  for (const [, buf] of primFunc.bufferMap) params.push(buf);
  const isZero = (p) => !!zeroData.get(params[p] && params[p].name);
  const epilogue = ew().matchEpilogue(tr, isZero);
  return { op: 'ewise', prog: tr.prog, inputIdx: tr.inputIdx, inNumel: tr.inNumel, outIdx: tr.outIdx,
           outNumel: tr.outNumel, outputIndices: [tr.outIdx], epilogue };
}

/** registerExternalCodegenProvider(...) entry (external_codegen.ts:11-17). */
function createHipProvider(EXTERNAL_CODEGEN_ATTR, CONST_BUFFERS_ATTR) {
  const attr = EXTERNAL_CODEGEN_ATTR || 'external_codegen';    // FuncAttr.EXTERNAL_CODEGEN
  const cattr = CONST_BUFFERS_ATTR || 'const_buffers';         // FuncAttr.CONST_BUFFERS
  return {
    name: PROVIDER,
    enabled(config, target) {
      const t = target && (target.kind || (target.features && target.features.kind));
      return t === HIP_KIND && !!(config && config.quantization && config.quantization.enabled);
    },
    annotate(tirModule) {
      for (const primFunc of tirModule) {
        const cbs = typeof primFunc.getAttr === 'function' ? primFunc.getAttr(cattr) : null;
        const info = describe(primFunc, cbs);
        if (info) primFunc.setAttr(attr, { name: PROVIDER, info });
      }
    },
  };
}

/**
 * Codegen entry for target kind 'hip' (registerCodegen,
 * codegen_registry.ts:26-28).  BackendPipeline.compile consults it for every
 * PrimFunc the provider did not tag (backend/pipeline.ts:46-47): ops outside
 * the int8 path that are not elementwise loop nests (reductions, softmax,
 * gathers).  They go to the target's host codegen entry -- the CPU one by
 * default -- and run on the JS runtime; the kernel's metadata records
 * hipRoute: 'host' so callers can see which kernels left the GPU.
 */
function createHipCodegenEntry(getCodegenEntry, hostKind) {
  const host = hostKind || 'cpu';
  return {
    runtimeKind: 'js',
    compile(primFunc, target, pipeline) {
      const entry = getCodegenEntry(host);
      need(entry, `no codegen entry for the host target kind '${host}'`);
      const out = entry.compile(primFunc, target, pipeline);
      out.metadata.hipRoute = 'host';
      return out;
    },
  };
}

/**
 * A compile target of kind 'hip'.  With the reference's target factory
 * (CPUTarget, support/target.ts:187-205) it is a real TargetFeatures whose
 * scheduling and layout choices are the host's (isGPU() is false for a
 * kind other than cuda / webgpu, so no thread binding is planned for the
 * host-routed kernels); int8 and constant buffers are supported.  Without
 * one, a plain object with the fields the provider and QuantizationPass
 * read.
 */
function hipTarget(CPUTarget, overrides, q8opts) {
  const f = { kind: HIP_KIND, name: 'hip_mi355x', supportsInt8: true, supportsConstBuffers: true };
  const mode = (q8opts && q8opts.activations) || 'static';
  need(ACTIVATION_MODES.has(mode), `q8 activations must be one of ${[...ACTIVATION_MODES].join(', ')} (got '${mode}')`);
  let t;
  if (typeof CPUTarget === 'function') {
    t = CPUTarget(Object.assign(f, overrides || {}));
  } else {
    const attrs = new Map();
    t = Object.assign({ isGPU: () => false, isCPU: () => false, attrs,
                        getAttr: (k, fb = null) => (attrs.has(k) ? attrs.get(k) : fb),
                        withAttr(k, v) { attrs.set(k, v); return this; } }, f, overrides || {});
  }
  if (mode !== 'static') {
    need(typeof t.withAttr === 'function', 'the target factory gives no withAttr for the q8 activation mode');
    t.withAttr(ACTIVATIONS_ATTR, mode);
  }
  return t;
}

/** The activation quantization a target asks for (ACTIVATIONS_ATTR). */
function activationMode(target) {
  const m = target && typeof target.getAttr === 'function' ? target.getAttr(ACTIVATIONS_ATTR) : null;
  if (m === null || m === undefined) return 'static';
  need(ACTIVATION_MODES.has(m), `unknown q8 activation mode '${m}'`);
  return m;
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
 * registerExternalCodegenProvider, registerCodegen?, getCodegenEntry?,
 * FuncAttr?, Library?, DispatchKey?, tensors? }.  With registerCodegen and
 * getCodegenEntry it also registers the 'hip' codegen entry, so the PrimFuncs
 * the provider leaves untagged compile for the host instead of throwing
 * 'Unsupported target kind: hip' (backend/pipeline.ts:46-47).
 */
/**
 * Kernel measurer of backend kind 'hip' (registerMeasurer('hip', ...), as
 * the reference registers one per runtime: measurer_registry.ts:5-15,
 * 'cuda' at cuda_runtime.ts:46-76,452; read by the autotuner,
 * autotuner.ts:80-88).  Same contract as measureCudaKernel: device buffers
 * of bufferByteSizes (the kernel's tensor arguments, then its constant
 * buffers) hold the arguments, `warmup` launches (and at least minWarmupMs
 * of them) run first, then `repeat` samples in milliseconds.  Each sample
 * is one launch of the descriptor's kernels and a synchronization of the
 * addon's stream, timed on the host: the device time of the launch plus
 * the host round trip (CUDA's samples time the asynchronous launch only).
 * Sizes below what the descriptor reads or writes are rejected.
 */
function measureHipKernel(kernel, bufferByteSizes, shapeValues, opts) {
  const d = kernel && kernel.metadata && kernel.metadata.q8;
  need(kernel && kernel.metadata && kernel.metadata.kind === HIP_KIND && d, 'measureHipKernel: not a hip kernel');
  need(!shapeValues || shapeValues.length === 0, 'dynamic shapes are not supported by the int8 kernels');
  const o = opts || {};
  const warmup = o.warmup !== undefined ? o.warmup : 5;
  const repeat = o.repeat !== undefined ? o.repeat : 30;
  const minWarmupMs = o.minWarmupMs !== undefined ? o.minWarmupMs : 25;
  const maxWarmup = o.maxWarmup !== undefined ? o.maxWarmup : 100000;
  const specs = new Map([...inputSpecs(d), ...outputSpecs(d)]);
  for (const [i, spec] of specs) {
    const have = bufferByteSizes[i] || 0, want = spec.n * spec.ctor.BYTES_PER_ELEMENT;
    need(have >= want, `measureHipKernel: buffer ${i} (${spec.what}) has ${have} bytes, the kernel needs ${want}`);
  }
  const A = q8();
  const dev = new DeviceArgs();
  const dv = bufferByteSizes.map((bytes, i) => dev.get(`m${i}`, Math.max(bytes, 1)));
  const now = () => Number(process.hrtime.bigint()) / 1e6;
  try {
    const once = () => execDevice(d, dv, dev, null);
    const t0 = now();
    for (let w = 0; w < maxWarmup && (w < warmup || now() - t0 < minWarmupMs); w++) once();
    A.sync();
    const samples = [];
    for (let i = 0; i < repeat; i++) {
      const a = now();
      once();
      A.sync();
      samples.push(now() - a);
    }
    return samples;
  } finally {
    dev.release();
  }
}

function registerHip(r) {
  need(r && typeof r.registerBackend === 'function', 'registerBackend is required');
  const fa = r.FuncAttr || {};
  r.registerBackend(HIP_KIND, createHipRuntimeBackend());
  if (r.registerMeasurer) r.registerMeasurer(HIP_KIND, measureHipKernel);
  if (r.registerExternalCodegen) r.registerExternalCodegen(PROVIDER, createHipExternalCodegen(fa.CONST_BUFFERS));
  if (r.registerExternalCodegenProvider) {
    r.registerExternalCodegenProvider(createHipProvider(fa.EXTERNAL_CODEGEN, fa.CONST_BUFFERS));
  }
  if (r.registerCodegen && r.getCodegenEntry) {
    r.registerCodegen(HIP_KIND, createHipCodegenEntry(r.getCodegenEntry, r.hostKind));
  }
  let library = null;
  if (r.Library && r.DispatchKey && r.tensors) library = defineEagerLibrary(r.Library, r.DispatchKey, r.tensors);
  return { kind: HIP_KIND, provider: PROVIDER, library };
}

module.exports = {
  HIP_KIND, PROVIDER, ACTIVATIONS_ATTR, activationMode, registerHip, createHipRuntimeBackend, createHipExternalCodegen, createHipCodegenEntry,
  createHipProvider, defineEagerLibrary, detectInt8Kernel, describe, runDescriptor, hipTarget, DeviceArgs,
  markHostDirty, stats, resetStats, setHipGraphEnabled, isHipGraphEnabled, releasePlan, measureHipKernel,
  // runPlan's body without the promise: it throws where runPlan rejects
  runPlanSync: runPlanOnDevice,
};
