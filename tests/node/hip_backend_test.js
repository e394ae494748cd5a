'use strict';
/*
 * Node-side tests of mlfw_amd/node (run by tests/test_node_host.py).
 *   node hip_backend_test.js cpu          registration, TIR matching, errors (no GPU)
 *   node hip_backend_test.js gpu <dir>    C1 through the 'hip' runtime backend and the
 *                                          eager library; writes outputs into <dir>
 * Mock registries and TIR nodes follow the reference's shapes
 * (src/runtime/backend_registry.ts:14-32, src/backend/codegen_registry.ts:17-36,
 * src/compiler/pipeline/external_codegen.ts:11-35, src/dispatcher/library.ts:30-72,
 * node field names as read by src/backend/cpu/codegen.ts:428-552).
 */
const fs = require('fs');
const path = require('path');
const assert = require('assert');

const ROOT = path.join(__dirname, '..', '..');
const hip = require(path.join(ROOT, 'mlfw_amd', 'node', 'hip_backend.js'));

let failures = 0;
function test(name, fn) {
  try { fn(); console.log(`ok   ${name}`); } catch (e) { failures++; console.log(`FAIL ${name}\n     ${e.stack}`); }
}

// ---------------------------------------------------------------- mocks
function makeRegistries() {
  const backends = new Map(), codegens = new Map(), providers = new Map(), ops = [], impls = new Map();
  class Library {
    constructor(ns, kind) { this.ns = ns; this.kind = kind; }
    def(schema) { ops.push(`${this.ns}::${schema}`); return this; }
    impl(name, key, fn) { impls.set(`${this.ns}::${name}`, { key, fn }); return this; }
  }
  const measurers = new Map();
  return {
    backends, codegens, providers, ops, impls, measurers,
    registerBackend: (k, b) => backends.set(k, b),
    registerMeasurer: (k, fn) => measurers.set(k, fn),
    registerExternalCodegen: (n, e) => codegens.set(n, e),
    registerExternalCodegenProvider: (p) => providers.set(p.name, p),
    FuncAttr: { EXTERNAL_CODEGEN: 'external_codegen' },
    Library, DispatchKey: { CPU: 0, GPU: 1 },
    tensors: { data: (t) => t.data, shape: (t) => t.shape, make: (data, shape) => ({ data, shape }) },
  };
}

const V = (name) => ({ type: 'VariableNode', name });
const F = (value) => ({ type: 'FloatImmNode', value });
const I = (value) => ({ type: 'IntImmNode', value });
const buf = (name, shape, dtype) => ({ name, shape, dtype });
const load = (b, idx) => ({ type: 'BufferLoadNode', buffer: b, indices: idx });
const ext = (externName, args) => ({ type: 'CallExternNode', externName, args });
const math = (op, a, b) => ({ type: 'MathOpNode', op, a, b });
const cast = (expr, toDtype, fromDtype = 'i8') => ({ type: 'CastNode', expr, fromDtype, toDtype });
function primFunc(name, params, blocks) {
  const attrs = {};
  const bufferMap = new Map(params.map((b, i) => [`v${i}`, b]));
  let body = blocks.length === 1 ? blocks[0] : { type: 'SeqNode', stmts: blocks };
  body = { type: 'ForNode', body };
  return { name, params, bufferMap, body, attrs, setAttr(k, v) { attrs[k] = v; return this; } };
}
function quantizePF(scale, zp, tgt) {
  const x = buf('x', [32, 128], 'f32'), q = buf('q', [32, 128], tgt);
  let e = math('/', load(x, [V('i'), V('j')]), F(scale));
  if (zp !== 0) e = math('+', e, F(zp));
  const value = cast(ext('min', [ext('max', [ext('round', [e]), F(tgt === 'ui8' ? 0 : -128)]), F(tgt === 'ui8' ? 255 : 127)]), tgt);
  const block = { type: 'BlockNode', name: 'quantize_block_0', reads: [{ buffer: x }], writes: [{ buffer: q }],
                  body: { type: 'BufferStoreNode', buffer: q, indices: [V('i'), V('j')], value } };
  return primFunc('quant', [x, q], [block]);
}
function dequantizePF(scale, zp, src) {
  const q = buf('q', [32, 128], src), y = buf('y', [32, 128], 'f32');
  let e = cast(load(q, [V('i'), V('j')]), 'f32');
  if (zp !== 0) e = math('-', e, F(zp));
  const block = { type: 'BlockNode', name: 'dequantize_block', reads: [{ buffer: q }], writes: [{ buffer: y }],
                  body: { type: 'BufferStoreNode', buffer: y, indices: [V('i'), V('j')], value: math('*', e, F(scale)) } };
  return primFunc('deq', [q, y], [block]);
}
function qdotPF(M, N, K, layout, zpA, zpB, aD = 'i8', bD = 'i8') {
  const a = buf('a', [M, K], aD), b = buf('b', layout === 'KN' ? [K, N] : [N, K], bD), c = buf('c', [M, N], 'i32');
  const m = V('m'), n = V('n'), k = V('k');
  let la = cast(load(a, [m, k]), 'i32', aD), lb = cast(load(b, layout === 'KN' ? [k, n] : [n, k]), 'i32', bD);
  if (zpA) la = math('-', la, I(zpA));
  if (zpB) lb = math('-', lb, I(zpB));
  const init = { type: 'BlockNode', name: 'qmatmul_init', reads: [], writes: [{ buffer: c }],
                 body: { type: 'BufferStoreNode', buffer: c, indices: [m, n], value: I(0) } };
  const acc = { type: 'BlockNode', name: 'qmatmul_acc_1', reads: [{ buffer: a }, { buffer: b }], writes: [{ buffer: c }],
                body: { type: 'BufferStoreNode', buffer: c, indices: [m, n],
                        value: math('+', load(c, [m, n]), math('*', la, lb)) } };
  return primFunc('qdot', [a, b, c], [init, acc]);
}

// mathOp's constant folding (src/compiler/ir/tensor/nodes.ts:394-430)
function mop(op, a, b) {
  if (a.type === 'IntImmNode' && b.type === 'IntImmNode') {
    if (op === '+') return I(a.value + b.value);
    if (op === '*') return I(a.value * b.value);
  }
  if (b.type === 'IntImmNode' && ((op === '+' && b.value === 0) || (op === '*' && b.value === 1))) return a;
  if (a.type === 'IntImmNode' && ((op === '+' && a.value === 0) || (op === '*' && a.value === 1))) return b;
  return math(op, a, b);
}
// qconv_init / qconv_acc as buildConvNest emits them
// (src/compiler/passes/lowering/lowering_registry.ts:335-449), NCHW / OIHW.
function qconvPF(xs, ws, strides, padding, dilation, groups) {
  const d = strides.length;
  const os = [xs[0], ws[0]];
  for (let s = 0; s < d; s++) {
    const eff = (ws[2 + s] - 1) * dilation[s] + 1;
    os.push(Math.floor((xs[2 + s] + padding[s][0] + padding[s][1] - eff) / strides[s]) + 1);
  }
  const x = buf('x', xs, 'i8'), w = buf('w', ws, 'i8'), y = buf('y', os, 'i32');
  const n = V('qcv0'), oc = V('qcv1'), ic = V(`qcv${2 + d}`);
  const so = [], sk = [];
  for (let s = 0; s < d; s++) { so.push(V(`qcv${2 + s}`)); sk.push(V(`qcv${3 + d + s}`)); }
  const Cg = ws[1], Og = ws[0] / groups;
  const inIdx = [n, groups > 1 ? math('+', math('*', math('//', oc, I(Og)), I(Cg)), ic) : ic];
  const kerIdx = [oc, ic];
  let bounds = null;
  for (let s = 0; s < d; s++) {
    const e = mop('+', mop('*', so[s], I(strides[s])), mop('+', mop('*', sk[s], I(dilation[s])), I(-padding[s][0])));
    inIdx.push(e);
    kerIdx.push(sk[s]);
    if (padding[s][0] || padding[s][1]) {
      const ok = math('*', { type: 'CompareNode', op: 'ge', a: e, b: I(0) }, { type: 'CompareNode', op: 'lt', a: e, b: I(xs[2 + s]) });
      bounds = bounds ? math('*', bounds, ok) : ok;
    }
  }
  const outIdx = [n, oc, ...so];
  const prod = math('*', cast(load(x, inIdx), 'i32'), cast(load(w, kerIdx), 'i32'));
  const guarded = bounds ? { type: 'IfThenElseNode', condition: bounds, thenBody: prod, elseBody: I(0) } : prod;
  const init = { type: 'BlockNode', name: 'qconv_init', reads: [], writes: [{ buffer: y }],
                 body: { type: 'BufferStoreNode', buffer: y, indices: outIdx, value: I(0) } };
  const acc = { type: 'BlockNode', name: 'qconv_acc_2', reads: [{ buffer: x }, { buffer: w }], writes: [{ buffer: y }],
                body: { type: 'BufferStoreNode', buffer: y, indices: outIdx, value: math('+', load(y, outIdx), guarded) } };
  return primFunc('qconv', [x, w, y], [init, acc]);
}
const CONV_CASE = { xs: [2, 4, 9, 7], ws: [6, 2, 3, 2], strides: [2, 1], padding: [[1, 2], [0, 1]],
                    dilation: [2, 1], groups: 2 };

// ---------------------------------------------------------------- CPU tests
function cpuTests() {
  test('detects quantized_conv geometry from the index expressions', () => {
    const c = CONV_CASE;
    const d = hip.detectInt8Kernel(qconvPF(c.xs, c.ws, c.strides, c.padding, c.dilation, c.groups));
    assert.ok(d);
    assert.strictEqual(d.op, 'quantized_conv');
    assert.deepStrictEqual([d.strides, d.padLo, d.dilation, d.groups], [[2, 1], [1, 0], [2, 1], 2]);
    assert.deepStrictEqual(d.outShape, [2, 6, 4, 7]);
    // the trailing padding is the smallest that yields the output size
    assert.deepStrictEqual(d.padHi, [1, 1]);
    // stride 1, dilation 1 and no padding fold to bare variables (x*1, +0)
    const e = hip.detectInt8Kernel(qconvPF([1, 3, 8, 8], [16, 3, 3, 3], [1, 1], [[0, 0], [0, 0]], [1, 1], 1));
    assert.deepStrictEqual([e.strides, e.padLo, e.padHi, e.dilation, e.groups], [[1, 1], [0, 0], [0, 0], [1, 1], 1]);
    const f = hip.detectInt8Kernel(qconvPF([1, 2, 10], [4, 2, 3], [3], [[2, 2]], [1], 1));
    assert.deepStrictEqual([f.d, f.strides, f.padLo, f.outShape], [1, [3], [2], [1, 4, 4]]);
  });

  test('registerHip plugs into all three registries', () => {
    const r = makeRegistries();
    const res = hip.registerHip(r);
    assert.strictEqual(res.kind, 'hip');
    const be = r.backends.get('hip');
    for (const k of ['instantiate', 'runSync', 'runAsync', 'isAsync']) assert.strictEqual(typeof be[k], 'function', k);
    assert.strictEqual(be.isAsync(), false);
    const cg = r.codegens.get('hip_int8');
    assert.strictEqual(cg.runtimeKind, 'hip');
    const out = cg.compile({ params: [] }, hip.hipTarget(), { op: 'quantize', outputIndices: [1] });
    assert.strictEqual(out.source, '');
    assert.deepStrictEqual(out.metadata.outputIndices, [1]);
    assert.strictEqual(out.metadata.kind, 'hip');
    assert.ok(r.ops.some((s) => s.startsWith('q8::quantize_per_token(')));
    assert.strictEqual(r.impls.get('q8::qlinear').key, 1);
    // the autotuner's measurer for kind 'hip' (measurer_registry.ts:5-15)
    assert.strictEqual(r.measurers.get('hip'), hip.measureHipKernel);
    const k = cg.compile({ params: [] }, hip.hipTarget(), { op: 'quantize', n: 64, scale: 0.1, zeroPoint: 0,
                                                            targetDtype: 'i8', inIdx: 0, outIdx: 1, outputIndices: [1] });
    assert.throws(() => hip.measureHipKernel(k, [4 * 64, 63], [], { repeat: 1 }), /buffer 1 .* has 63 bytes, the kernel needs 64/);
  });

  test('provider is enabled only for the hip target with quantization on', () => {
    const p = hip.createHipProvider();
    assert.strictEqual(p.enabled({ quantization: { enabled: true } }, hip.hipTarget()), true);
    assert.strictEqual(p.enabled({ quantization: { enabled: false } }, hip.hipTarget()), false);
    assert.strictEqual(p.enabled({ quantization: { enabled: true } }, { kind: 'cuda' }), false);
  });

  test('detects quantize with its static scale, zero point and target dtype', () => {
    const d = hip.detectInt8Kernel(quantizePF(6 / 127, 0, 'i8'));
    assert.deepStrictEqual(d, { op: 'quantize', n: 4096, scale: 6 / 127, zeroPoint: 0, targetDtype: 'i8',
                                inIdx: 0, outIdx: 1, outputIndices: [1] });
    const u = hip.detectInt8Kernel(quantizePF(1 / 255, 3, 'ui8'));
    assert.strictEqual(u.zeroPoint, 3);
    assert.strictEqual(u.targetDtype, 'ui8');
  });

  test('detects dequantize from i8, ui8 and i32', () => {
    for (const src of ['i8', 'ui8', 'i32']) {
      const d = hip.detectInt8Kernel(dequantizePF(0.02, src === 'ui8' ? 128 : 0, src));
      assert.strictEqual(d.op, 'dequantize');
      assert.strictEqual(d.srcDtype, src);
      assert.strictEqual(d.scale, 0.02);
    }
  });

  test('detects quantized_dot layout from the reduction index, also when square', () => {
    for (const [M, N, K] of [[32, 64, 128], [64, 64, 64]]) {
      for (const layout of ['NK', 'KN']) {
        const d = hip.detectInt8Kernel(qdotPF(M, N, K, layout, 0, 0));
        assert.ok(d, `${layout} ${M}x${N}x${K}`);
        assert.strictEqual(d.rhsLayout, layout);
        assert.deepStrictEqual([d.M, d.N, d.K, d.aIdx, d.bIdx, d.outIdx], [M, N, K, 0, 1, 2]);
      }
    }
    const z = hip.detectInt8Kernel(qdotPF(8, 8, 16, 'NK', 3, -2));
    assert.deepStrictEqual([z.zpA, z.zpB], [3, -2]);
    // ui8 operands (an affine activation scheme: zero point 128)
    const u = hip.detectInt8Kernel(qdotPF(8, 8, 16, 'KN', 128, 0, 'ui8', 'i8'));
    assert.deepStrictEqual([u.zpA, u.zpB, u.aDtype, u.bDtype, u.rhsLayout], [128, 0, 'ui8', 'i8', 'KN']);
  });

  test('annotate tags only the int8 PrimFuncs', () => {
    const p = hip.createHipProvider('external_codegen');
    const funcs = [quantizePF(0.1, 0, 'i8'), qdotPF(4, 4, 16, 'NK', 0, 0),
                   primFunc('other', [buf('a', [4], 'f32')], [{ type: 'BlockNode', name: 'add_block', reads: [], writes: [], body: null }])];
    p.annotate(funcs);
    assert.strictEqual(funcs[0].attrs.external_codegen.name, 'hip_int8');
    assert.strictEqual(funcs[1].attrs.external_codegen.info.op, 'quantized_dot');
    assert.strictEqual(funcs[2].attrs.external_codegen, undefined);
  });

  test('runtime backend validates descriptors before touching a device', () => {
    const be = hip.createHipRuntimeBackend();
    assert.throws(() => be.instantiate({ metadata: { kind: 'cuda' } }), /not hip/);
    assert.throws(() => be.instantiate({ metadata: { kind: 'hip' } }), /no q8 descriptor/);
    const inst = be.instantiate({ metadata: { kind: 'hip', q8: { op: 'quantize', n: 4, scale: 1, zeroPoint: 0,
                                                                 targetDtype: 'i8', inIdx: 0, outIdx: 1 } } });
    assert.throws(() => be.runSync(inst, [new Float64Array(4), new Int8Array(4)], null), /Float32Array/);
    assert.throws(() => be.runSync(inst, [new Float32Array(4), new Int8Array(4)], [7]), /dynamic shapes/);
  });

  test('the addon loads and reports errors as coded exceptions', () => {
    const a = require(path.join(ROOT, 'mlfw_amd', 'node', 'index.js'));
    assert.strictEqual(a.version(), 1);
    assert.ok(a.deviceCount() >= 0);
    assert.throws(() => a.quantizeStatic(null, 10, 0.0, 0, a.Q8_I8, null), (e) => e.code === 'Q8_ERR_1');
    assert.throws(() => a.gemm(null, null, 4, 4, 16, 0, 0, null, 0, null, 0, 9, 0, null, 0, a.Q8_F32, null),
                  (e) => e.code === 'Q8_ERR_1' && /bad epi/.test(e.message));
    assert.throws(() => a.upload({}, new Float32Array(1)), TypeError);
    for (const f of ['gemmRequant', 'packWeightInt4', 'gemvW4', 'qlinearDynamic', 'quantizedDot',
                     'quantizedDotWorkspace', 'quantizedConvEx']) assert.strictEqual(typeof a[f], 'function', f);
    assert.strictEqual(a.quantizedDotWorkspace(4, 5, 16, a.Q8_U8, a.Q8_I8, 128, 0), 256);
    assert.throws(() => a.quantizedDot(null, 7, null, a.Q8_I8, 4, 5, 16, 0, 0, null, null),
                  (e) => e.code === 'Q8_ERR_1');
    assert.throws(() => a.qlinearDynamic(null, 1, 16, 9, null, null, 0, 4, null, 0, null, null, null),
                  (e) => e.code === 'Q8_ERR_1' && /x_mode/.test(e.message));
    assert.throws(() => a.gemvW4(null, null, a.Q8_PER_TOKEN, null, null, 1, 4, 96, 64, null, 0, null),
                  (e) => e.code === 'Q8_ERR_1' && /group_size/.test(e.message));
    assert.throws(() => a.packWeightInt4(null, 4, 96, 7, null, null), (e) => e.code === 'Q8_ERR_1');
    assert.throws(() => a.gemmRequant(null, null, 4, 4, 16, null, 0, null, 0, 9, 0, null, 0, 0.1, null),
                  (e) => e.code === 'Q8_ERR_1');
  });

  test('runtime backend validates the requant and W4 descriptors', () => {
    const be = hip.createHipRuntimeBackend();
    const rq = be.instantiate({ metadata: { kind: 'hip', q8: { op: 'qlinear_requant', M: 2, N: 4, K: 16, xqIdx: 0,
                                                               sxIdx: 1, wqIdx: 2, wsIdx: 3, outIdx: 4, sNext: 0.1 } } });
    assert.throws(() => be.runSync(rq, [new Int8Array(32), new Float64Array(2), new Int8Array(64),
                                        new Float64Array(4), new Float32Array(8)], null), /qlinear_requant out/);
    const w4 = be.instantiate({ metadata: { kind: 'hip', q8: { op: 'qlinear_w4', M: 1, N: 4, K: 64, group: 32,
                                                               xIdx: 0, wqIdx: 1, swIdx: 2, outIdx: 3 } } });
    assert.throws(() => be.runSync(w4, [new Float32Array(64), new Int8Array(128), new Float64Array(8),
                                        new Float32Array(4)], null), /packed weights/);
  });
}

// ---------------------------------------------------------------- GPU tests
function readArr(dir, name, T) {
  const b = fs.readFileSync(path.join(dir, name));
  return new T(b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength));
}
function writeArr(dir, name, a) {
  fs.writeFileSync(path.join(dir, name), Buffer.from(a.buffer, a.byteOffset, a.byteLength));
}

function gpuTests(dir) {
  const a = require(path.join(ROOT, 'mlfw_amd', 'node', 'index.js'));
  a.init(0);
  const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json')));
  const X = readArr(dir, 'X.bin', Float32Array), Xq = readArr(dir, 'Xq.bin', Int8Array);
  const Wq = readArr(dir, 'Wq.bin', Int8Array), sW = readArr(dir, 'sW.bin', Float64Array);
  const bias = readArr(dir, 'bias.bin', Float32Array);
  const { M, N, K, sX } = meta;
  const r = makeRegistries();
  hip.registerHip(r);
  const be = r.backends.get('hip');
  const cg = r.codegens.get('hip_int8');

  test('measurer for kind hip: per-launch samples in milliseconds', () => {
    const kern = cg.compile({}, hip.hipTarget(), { op: 'quantized_dot', M: 64, N: 256, K: 512, aIdx: 0, bIdx: 1,
                                                   outIdx: 2, rhsLayout: 'NK', zpA: 0, zpB: 0, outputIndices: [2] });
    const samples = r.measurers.get('hip')(kern, [64 * 512, 256 * 512, 4 * 64 * 256], [], { warmup: 2, repeat: 7, minWarmupMs: 1 });
    assert.strictEqual(samples.length, 7);
    for (const t of samples) assert.ok(t > 0 && t < 1000, `sample ${t} ms`);
  });

  test('runtime backend: compiled quantize (static scale) on the GPU', () => {
    const kern = cg.compile({}, hip.hipTarget(), { op: 'quantize', n: M * K, scale: sX, zeroPoint: 0,
                                                   targetDtype: 'i8', inIdx: 0, outIdx: 1, outputIndices: [1] });
    const inst = be.instantiate(kern);
    const q = new Int8Array(M * K);
    be.runSync(inst, [X, q], null);
    writeArr(dir, 'out_quantize.bin', q);
  });

  test('runtime backend: quantized_dot [N,K] and [K,N] weights on the GPU', () => {
    for (const layout of ['NK', 'KN']) {
      let B = Wq;
      if (layout === 'KN') { B = new Int8Array(K * N); for (let n = 0; n < N; n++) for (let k = 0; k < K; k++) B[k * N + n] = Wq[n * K + k]; }
      const kern = cg.compile({}, hip.hipTarget(), { op: 'quantized_dot', M, N, K, rhsLayout: layout, zpA: 0, zpB: 0,
                                                     aIdx: 0, bIdx: 1, outIdx: 2, outputIndices: [2] });
      const acc = new Int32Array(M * N);
      be.runSync(be.instantiate(kern), [Xq, B, acc], null);
      writeArr(dir, `out_qdot_${layout}.bin`, acc);
    }
  });

  test('runtime backend: quantized_dot with a ui8 operand and zero points on the GPU', () => {
    const Au = readArr(dir, 'qdot_u8_a.bin', Uint8Array);
    const kern = cg.compile({}, hip.hipTarget(), { op: 'quantized_dot', M, N, K, rhsLayout: 'NK', zpA: 128, zpB: 3,
                                                   aDtype: 'ui8', bDtype: 'i8', aIdx: 0, bIdx: 1, outIdx: 2,
                                                   outputIndices: [2] });
    const acc = new Int32Array(M * N);
    be.runSync(be.instantiate(kern), [Au, Wq, acc], null);
    writeArr(dir, 'out_qdot_u8.bin', acc);
  });

  test('runtime backend: dequantize of int32 accumulators (per-tensor epilogue E-pt)', () => {
    const acc = readArr(dir, 'out_qdot_NK.bin', Int32Array);
    const kern = cg.compile({}, hip.hipTarget(), { op: 'dequantize', n: M * N, scale: meta.sOut, zeroPoint: 0,
                                                   srcDtype: 'i32', inIdx: 0, outIdx: 1, outputIndices: [1] });
    const y = new Float32Array(M * N);
    be.runSync(be.instantiate(kern), [acc, y], null);
    writeArr(dir, 'out_dequant_i32.bin', y);
  });

  test('runtime backend: fused qlinear (C1: per-tensor dynamic quantize + GEMM + per-channel epilogue + bias)', () => {
    const y = new Float32Array(M * N);
    const inst = be.instantiate({ metadata: { kind: 'hip', q8: { op: 'qlinear', M, N, K, xIdx: 0, wqIdx: 1, wsIdx: 2,
                                                                  biasIdx: 3, outIdx: 4, granularity: 'per_tensor', act: 'none' } } });
    be.runSync(inst, [X, Wq, sW, bias, y], null);
    writeArr(dir, 'out_c1.bin', y);
  });

  test('eager library: q8::quantize_per_token and q8::dequantize_per_token', () => {
    const qpt = r.impls.get('q8::quantize_per_token').fn;
    const dpt = r.impls.get('q8::dequantize_per_token').fn;
    const [q, s] = qpt({ data: X, shape: [M, K] });
    writeArr(dir, 'out_qpt_q.bin', q.data);
    writeArr(dir, 'out_qpt_s.bin', s.data);
    const y = dpt(q, s);
    assert.deepStrictEqual(y.shape, [M, K]);
    writeArr(dir, 'out_dpt.bin', y.data);
  });

  test('runtime backend: quantized_conv PrimFunc on the GPU', () => {
    const c = CONV_CASE;
    const xc = readArr(dir, 'conv_x.bin', Int8Array), wc = readArr(dir, 'conv_w.bin', Int8Array);
    const pf = qconvPF(c.xs, c.ws, c.strides, c.padding, c.dilation, c.groups);
    const info = hip.detectInt8Kernel(pf);
    const kern = cg.compile(pf, hip.hipTarget(), info);
    const y = new Int32Array(info.outShape.reduce((a, b) => a * b, 1));
    be.runSync(be.instantiate(kern), [xc, wc, y], null);
    writeArr(dir, 'out_conv.bin', y);
  });

  test('runtime backend: a constant conv weight is prepacked once and gives the same bits', () => {
    // 32 channels per group, 3 x 3: the channel-last path reads the tap-major form
    const xs = [2, 64, 9, 9], ws = [48, 32, 3, 3];
    const pf = qconvPF(xs, ws, [1, 1], [[1, 1], [1, 1]], [1, 1], 2);
    const info = hip.detectInt8Kernel(pf);
    const xc = new Int8Array(xs.reduce((a, b) => a * b, 1)), wc = new Int8Array(ws.reduce((a, b) => a * b, 1));
    for (let i = 0; i < xc.length; i++) xc[i] = ((i * 2654435761) >>> 24) - 128;
    for (let i = 0; i < wc.length; i++) wc[i] = ((i * 40503 + 17) >>> 8 & 255) - 128;
    const n = info.outShape.reduce((a, b) => a * b, 1);
    const plain = new Int32Array(n);
    be.runSync(be.instantiate(cg.compile(pf, hip.hipTarget(), info)), [xc, wc, plain], null);
    // the same op with the weight as the kernel's constant buffer (appended
    // after the tensor arguments, runtime.ts:246-258)
    const dConst = Object.assign({}, info, { xIdx: 0, outIdx: 1, wIdx: 2, outputIndices: [1] });
    const kConst = { metadata: { kind: 'hip', q8: dConst, constBuffers: [{ name: 'w', dtype: 'i8', data: wc }] } };
    const inst = be.instantiate(kConst);
    hip.resetStats();
    for (let call = 0; call < 2; call++) {
      const y = new Int32Array(n);
      be.runSync(inst, [xc, y, wc], null);
      assert.ok(Buffer.compare(Buffer.from(y.buffer), Buffer.from(plain.buffer)) === 0, `prepacked conv, call ${call}`);
    }
    assert.strictEqual(hip.stats.constUploadBytes, wc.byteLength, 'the weight is uploaded (and prepacked) once');
  });

  test('runtime backend: one-token dynamic qlinear (quantize + GEMV in one kernel)', () => {
    const y = new Float32Array(N);
    const inst = be.instantiate({ metadata: { kind: 'hip', q8: { op: 'qlinear', M: 1, N, K, xIdx: 0, wqIdx: 1, wsIdx: 2,
                                                                  biasIdx: 3, outIdx: 4, granularity: 'per_token',
                                                                  act: 'silu' } } });
    be.runSync(inst, [X.subarray(0, K), Wq, sW, bias, y], null);
    writeArr(dir, 'out_qlinear1.bin', y);
  });

  test('runtime backend: int8 linear with the fused static requant (int8 out)', () => {
    const sx = readArr(dir, 'sx_tok.bin', Float64Array), xq = readArr(dir, 'xq_tok.bin', Int8Array);
    const out = new Int8Array(M * N);
    const inst = be.instantiate({ metadata: { kind: 'hip', q8: { op: 'qlinear_requant', M, N, K, xqIdx: 0, sxIdx: 1,
                                                                  wqIdx: 2, wsIdx: 3, biasIdx: 4, outIdx: 5,
                                                                  act: 'relu', sNext: meta.sNext } } });
    be.runSync(inst, [xq, sx, Wq, sW, bias, out], null);
    writeArr(dir, 'out_requant.bin', out);
  });

  test('runtime backend: W4A8 decode linear (4-bit per-group weights)', () => {
    const wq4 = readArr(dir, 'w4_q.bin', Uint8Array), sw4 = readArr(dir, 'w4_s.bin', Float64Array);
    const xs = X.subarray(0, meta.w4M * K);
    const y = new Float32Array(meta.w4M * N);
    const inst = be.instantiate({ metadata: { kind: 'hip', q8: { op: 'qlinear_w4', M: meta.w4M, N, K,
                                                                  group: meta.w4Group, xIdx: 0, wqIdx: 1, swIdx: 2,
                                                                  biasIdx: 3, outIdx: 4, act: 'silu' } } });
    be.runSync(inst, [xs, wq4, sw4, bias, y], null);
    writeArr(dir, 'out_w4.bin', y);
  });

  test('async path resolves to the same result', () => {
    const kern = cg.compile({}, hip.hipTarget(), { op: 'quantize', n: M * K, scale: sX, zeroPoint: 0,
                                                   targetDtype: 'i8', inIdx: 0, outIdx: 1, outputIndices: [1] });
    const q = new Int8Array(M * K);
    return be.runAsync(be.instantiate(kern), [X, q], null);
  });
}

const mode = process.argv[2];
if (mode === 'cpu') cpuTests();
else if (mode === 'gpu') gpuTests(process.argv[3]);
else { console.error('usage: hip_backend_test.js cpu | gpu <dir>'); process.exit(2); }
if (failures) { console.log(`${failures} failed`); process.exit(1); }
console.log('all passed');
