'use strict';
/*
 * Elementwise PrimFuncs and whole-plan execution on the 'hip' target
 * (run by tests/test_node_ewise.py).
 *   node ewise_test.js cpu    oracle pinning, translation, epilogue matching,
 *                             compile routing (no GPU)
 *   node ewise_test.js gpu    every PrimFunc through runSync, and the per-channel
 *                             Linear + bias + ReLU PrimFunc set through runPlan
 *                             (fused and unfused), bit for bit against the oracle
 * TIR nodes are plain objects with the reference's field names
 * (src/compiler/ir/tensor/nodes.ts); loop nests are built the way
 * lowerPointwise builds them (src/compiler/passes/lowering/lowering_registry.ts:
 * 277-306, 521-576): loop vars i_d, block iter vars v_d bound to them, loads
 * through computeBroadcastIndices.
 */
const path = require('path');
const assert = require('assert');

const ROOT = path.join(__dirname, '..', '..');
const hip = require(path.join(ROOT, 'mlfw_amd', 'node', 'hip_backend.js'));
const ew = require(path.join(ROOT, 'mlfw_amd', 'node', 'ewise.js'));
const ref = require(path.join(ROOT, 'oracle', 'ewise_ref.js'));        // the checker
const q8ref = require(path.join(ROOT, 'oracle', 'q8ref.js'));          // the checker

let failures = 0;
function test(name, fn) {
  try { fn(); console.log(`ok   ${name}`); } catch (e) { failures++; console.log(`FAIL ${name}\n     ${e.stack}`); }
}
// tests of a promise: settled before the process reports and exits
const pending = [];
function testAsync(name, promiseFn) {
  let p;
  try { p = Promise.resolve(promiseFn()); } catch (e) { p = Promise.reject(e); }
  pending.push(p.then(() => console.log(`ok   ${name}`),
                      (e) => { failures++; console.log(`FAIL ${name}\n     ${e && e.stack}`); }));
}

// ---------------------------------------------------------------- TIR builders
const { V, I, F, buf, load, math, ext, cast, cmp, sel, primFunc, pointwise, quantizeExpr, qmatmulPF } =
  require(path.join(ROOT, 'mlfw_amd', 'node', 'tir_build.js'));

// ---------------------------------------------------------------- data
function rng(seed) { return q8ref.makeRng(seed); }
function normal(seed, n, std = 1) { const a = new Float32Array(n); q8ref.normalFill(rng(seed), a, 0, std); return a; }
function withEdges(a) {
  const e = [NaN, Infinity, -Infinity, -0, 0, 0.5, -0.5, 2.5, -2.5, 1e-40, -1e-40, 3.4e38, -3.4e38, 127.5, -128.5];
  for (let i = 0; i < e.length && i < a.length; i++) a[(i * 7919) % a.length] = e[i];
  return a;
}
function randI8(seed, n) { const r = rng(seed), a = new Int8Array(n); for (let i = 0; i < n; i++) a[i] = Math.floor(r() * 256) - 128; return a; }
function randI32(seed, n, span) { const r = rng(seed), a = new Int32Array(n); for (let i = 0; i < n; i++) a[i] = Math.floor((r() - 0.5) * span); return a; }

function sameBits(got, want, what) {
  assert.strictEqual(got.length, want.length, `${what}: length`);
  const isF = got instanceof Float32Array || got instanceof Float64Array;
  let bad = 0, first = -1;
  for (let i = 0; i < got.length; i++) {
    const g = got[i], w = want[i];
    // a NaN stored into a float array may take any encoding (ECMA-262
    // NumericToRawBytes), so any NaN equals any NaN
    const eq = isF ? (Number.isNaN(g) && Number.isNaN(w)) || Object.is(g, w) : g === w;
    if (!eq) { bad++; if (first < 0) first = i; }
  }
  assert.strictEqual(bad, 0, `${what}: ${bad} of ${got.length} differ, first at ${first}: ${got[first]} vs ${want[first]}`);
}

// JS interpreter of a translated program (the device kernel's semantics), so
// the translation can be checked on the CPU against the oracle.
function emulate(tr, args) {
  const p = tr.prog, OP = ew.OP, out = args[tr.outIdx];
  const n = p.extent.reduce((a, b) => a * b, 1);
  const toI32 = (x) => x | 0;
  const jsmax = Math.max, jsmin = Math.min;
  const idx = new Array(6).fill(0);
  for (let e = 0; e < n; e++) {
    let rem = e;
    for (let d = p.ndims - 1; d >= 0; d--) { idx[d] = rem % p.extent[d]; rem = Math.floor(rem / p.extent[d]); }
    const R = new Array(16).fill(0);
    for (let pc = 0; pc < p.ncode; pc++) {
      const c = p.code[pc], a = R[c.a], b = R[c.b];
      let v;
      switch (c.op) {
        case OP.LOAD: { const j = c.aux; let off = p.inCoef[j][6]; for (let d = 0; d < 6; d++) off += p.inCoef[j][d] * idx[d]; v = args[tr.inputIdx[j]][off]; break; }
        case OP.CONST: v = p.konst[c.aux]; break;
        case OP.INDEX: v = idx[c.aux]; break;
        case OP.ADD: v = a + b; break;
        case OP.SUB: v = a - b; break;
        case OP.MUL: v = a * b; break;
        case OP.DIV: v = a / b; break;
        case OP.IDIV: v = Math.trunc(a / b); break;
        case OP.MOD: v = ((a % b + b) % b); break;
        case OP.FLOORDIV: v = Math.floor(a / b); break;
        case OP.TMOD: v = a % b; break;
        case OP.TDIV: v = (a / b) | 0; break;
        case OP.NEG: v = -a; break;
        case OP.CMP: v = [a === b, a !== b, a < b, a <= b, a > b, a >= b][c.aux] ? 1 : 0; break;
        case OP.SELECT: v = a ? b : R[c.c]; break;
        case OP.TOINT32: v = toI32(a); break;
        case OP.TOBOOL: v = a ? 1 : 0; break;
        case OP.MAX: v = jsmax(a, b); break;
        case OP.MIN: v = jsmin(a, b); break;
        case OP.ABS: v = Math.abs(a); break;
        case OP.FLOOR: v = Math.floor(a); break;
        case OP.CEIL: v = Math.ceil(a); break;
        case OP.ROUND: v = Math.round(a); break;
        case OP.SIGN: v = Math.sign(a); break;
        case OP.SQRT: v = Math.sqrt(a); break;
        case OP.FMOD: v = ((a % b + b) % b); break;
        case OP.EXP: v = Math.exp(a); break;
        case OP.LOG: v = Math.log(a); break;
        case OP.TANH: v = Math.tanh(a); break;
        case OP.RSQRT: v = 1.0 / Math.sqrt(a); break;
        case OP.POW: v = Math.pow(a, b); break;
        default: throw new Error(`op ${c.op}`);
      }
      if (c.rnd) v = Math.fround(v);
      R[c.dst] = v;
    }
    out[e] = R[p.result];
  }
}

// ---------------------------------------------------------------- the cases
const M = 37, N = 96, K = 256;
function linearSet(sX = 4.9 / 127) {
  const x = buf('x', [M, K], 'f32'), xq = buf('xq', [M, K], 'i8'), W = buf('w', [N, K], 'i8');
  const acc = buf('acc', [M, N], 'i32'), sv = buf('sv', [N], 'f32'), b = buf('b', [N], 'f32');
  const y = buf('y', [M, N], 'f32'), y2 = buf('y2', [M, N], 'f32'), y3 = buf('y3', [M, N], 'f32');
  const zero = buf('zero', [1, 1], 'f32'), q2 = buf('q2', [M, N], 'i8');
  const sNext = 0.0371;
  const Wdata = randI8(5, N * K);
  const svData = new Float32Array(N);
  for (let i = 0; i < N; i++) svData[i] = Math.fround(sX * (0.001 + 0.0002 * ((i * 37) % 17)));
  const consts = { W: { buffer: W, data: Wdata }, sv: { buffer: sv, data: svData },
                   zero: { buffer: zero, data: new Float32Array([0]) } };
  const pf = {
    quantize: pointwise('quantize', xq, [x], (l) => quantizeExpr(l[0], sX)),
    qmatmul: qmatmulPF(M, N, K, xq, W, acc, [consts.W]),
    tail: pointwise('fused_convert_mul', y, [acc, sv], (l) => math('*', cast(l[0], 'i32', 'f32'), l[1]), [consts.sv]),
    add: pointwise('add', y2, [y, b], (l) => math('+', l[0], l[1])),
    max: pointwise('maximum', y3, [y2, zero], (l) => ext('max', [l[0], l[1]]), [consts.zero]),
    fused: pointwise('fused_convert_mul_add_maximum', y3, [acc, sv, b, zero],
                     (l) => ext('max', [math('+', math('*', cast(l[0], 'i32', 'f32'), l[1]), l[2]), l[3]]),
                     [consts.sv, consts.zero]),
    reluQuant: pointwise('fused_maximum_quantize', q2, [y2, zero],
                         (l) => quantizeExpr(ext('max', [l[0], l[1]]), sNext), [consts.zero]),
    fusedRq: pointwise('fused_convert_mul_add_maximum_quantize', q2, [acc, sv, b, zero],
                       (l) => quantizeExpr(ext('max', [math('+', math('*', cast(l[0], 'i32', 'f32'), l[1]), l[2]), l[3]]),
                                           sNext), [consts.sv, consts.zero]),
  };
  return { bufs: { x, xq, W, acc, sv, b, y, y2, y3, zero, q2 }, pf, consts, sX, sNext };
}

// extra elementwise shapes: broadcasts, casts, compare/select, externs, lets
function extraCases() {
  const A = buf('a', [3, 5, 7], 'f32'), B = buf('b', [5, 1], 'f32'), C = buf('c', [7], 'f32');
  const O = buf('o', [3, 5, 7], 'f32'), OI = buf('oi', [3, 5, 7], 'i32'), OB = buf('ob', [3, 5, 7], 'ui8');
  const Q = buf('q', [3, 5, 7], 'i8'), D = buf('d', [3, 5, 7], 'f64');
  const cases = [
    ['broadcast add/mul chain', pointwise('fused', O, [A, B, C], (l) => math('*', math('+', l[0], l[1]), math('-', l[2], F(0.25))))],
    ['x - 0 and x * 1 folds', pointwise('fold', O, [A], (l) => math('+', math('*', math('-', l[0], I(0)), I(1)), F(0)))],
    ['silu', pointwise('silu', O, [A], (l) => math('*', l[0], math('/', F(1), math('+', F(1), ext('exp', [math('-', l[0])])))))],
    ['compare/select', pointwise('sel', O, [A, C], (l) => sel(cmp('gt', l[0], l[1]), l[0], math('*', l[1], F(2))))],
    ['cast to i32 (| 0)', pointwise('cvt', OI, [A], (l) => cast(math('*', l[0], F(1e9)), 'f32', 'i32'))],
    ['cast to bool', pointwise('cvtb', OB, [A], (l) => cast(l[0], 'f32', 'bool'))],
    ['exact externs', pointwise('ex', O, [A, C], (l) => ext('min', [ext('abs', [ext('floor', [math('*', l[0], F(3))])]),
                                                                    ext('sqrt', [ext('sign', [l[1]])])]))],
    ['round / ceil / fmod', pointwise('rnd', O, [A, C], (l) => math('+', ext('round', [math('*', l[0], F(2))]),
                                                                      ext('fmod', [ext('ceil', [l[0]]), F(3)])))],
    ['tanh / rsqrt / log / pow', pointwise('tr', O, [A], (l) => math('+', math('+', ext('tanh', [l[0]]), ext('rsqrt', [ext('abs', [l[0]])])),
                                                                   math('+', ext('log', [ext('abs', [l[0]])]), ext('pow', [ext('abs', [l[0]]), F(0.75)]))))],
    ['quantize ui8 with zero point', pointwise('q8u', OB, [A], (l) => quantizeExpr(l[0], 0.0123, 128, 'ui8'))],
    ['quantize i8', pointwise('q8', Q, [A], (l) => quantizeExpr(l[0], 0.02))],
    ['f64 output', pointwise('f64', D, [A, C], (l) => cast(math('*', l[0], l[1]), 'f32', 'f64'))],
    ['index arithmetic (iota)', pointwise('iota', OI, [], (l, ix) => math('+', math('*', ix[0], I(7)), math('-', ix[2], ix[1])))],
  ];
  return { cases, A, B, C };
}

function argsFor(pf, fill) {
  const args = [];
  for (const [, b] of pf.bufferMap) args.push(fill(b));
  return args;
}
function alloc(b) {
  const T = { f32: Float32Array, f64: Float64Array, i32: Int32Array, i8: Int8Array, ui8: Uint8Array }[b.dtype];
  return new T(b.shape.reduce((a, c) => a * c, 1));
}

// ---------------------------------------------------------------- CPU tests
function cpuTests() {
  // expected strings of tests/backend/cpu/codegen-internals.test.js
  test('oracle exprToJS reproduces the reference codegen-internals vectors', () => {
    const e = (n) => ref.exprToJS(n, new Map());
    const idx = (n) => V(n, 'index');
    const vectors = [
      [I(42), '42'], [I(0), '0'], [I(-7), '-7'], [F(3.14), '3.14'], [F(0), '0'], [F(-1.5), '-1.5'],
      [V('i0', 'index'), 'i0'], [math('+', I(3), I(4)), '(3 + 4)'], [math('*', idx('i'), I(8)), '(i * 8)'],
      [math('-', I(10), I(3)), '(10 - 3)'], [math('-', V('x', 'f32')), '(-x)'],
      [math('%', idx('x'), I(4)), '((x % 4 + 4) % 4)'], [math('//', idx('x'), I(4)), 'Math.floor(x / 4)'],
      [math('tdiv', idx('x'), I(4)), '((x / 4) | 0)'], [math('+', idx('x'), I(0)), 'x'], [math('+', I(0), idx('x')), 'x'],
      [math('+', V('x', 'f32'), I(0)), 'Math.fround(x + 0)'], [math('+', I(0), V('x', 'f32')), 'Math.fround(0 + x)'],
      [math('-', V('x', 'f32'), I(0)), 'x'], [math('*', idx('x'), I(0)), '0'], [math('*', I(0), idx('x')), '0'],
      [math('*', V('x', 'i64'), I(0)), '0n'], [math('*', V('x', 'f32'), I(0)), 'Math.fround(x * 0)'],
      [math('*', I(0), V('x', 'f32')), 'Math.fround(0 * x)'], [math('*', V('x', 'f32'), I(1)), 'x'],
      [math('*', I(1), V('x', 'f32')), 'x'], [math('*', math('+', idx('i'), I(1)), I(4)), '((i + 1) * 4)'],
      [cmp('ge', idx('x'), I(0)), '(x >= 0)'], [cmp('eq', idx('a'), idx('b')), '(a === b)'],
      [sel(cmp('gt', V('x', 'f32'), I(0)), F(1), F(0)), '((x > 0) ? 1 : 0)'],
      [cast(F(3.7), 'f32', 'i32'), '(3.7 | 0)'], [cast(I(5), 'i32', 'f32'), '(+5)'], [cast(idx('x'), 'index', 'bool'), '(x ? 1 : 0)'],
      [ext('exp', [V('x', 'f32')], 'f32'), 'Math.fround(Math.exp(x))'], [ext('sqrt', [V('x', 'f32')], 'f32'), 'Math.sqrt(x)'],
      [ext('rsqrt', [V('x', 'f32')], 'f32'), 'Math.fround(1.0 / Math.sqrt(x))'],
      [ext('max', [V('a', 'f32'), V('b', 'f32')], 'f32'), 'Math.max(a, b)'],
      [ext('fmod', [V('a', 'f32'), V('b', 'f32')], 'f32'), '((a % b + b) % b)'],
      [load(buf('buf_1', [4], 'f32'), [V('i', 'index')]), 'buf_1[i]'],
    ];
    for (const [node, want] of vectors) assert.strictEqual(e(node), want);
    assert.throws(() => e(ext('fake_func', [V('x', 'f32')], 'f32')), /unsupported extern function "fake_func"/);
    assert.strictEqual(e(null), '0');
    // _flatIndex vectors
    const fi = (b, ix) => ref.flatIndex(b, ix, new Map());
    assert.strictEqual(fi(buf('s', [], 'f32'), []), '0');
    assert.strictEqual(fi(buf('v', [8], 'f32'), [idx('i')]), 'i');
    assert.strictEqual(fi(buf('m', [3, 4], 'f32'), [idx('i'), idx('j')]), 'i * 4 + j');
    assert.strictEqual(fi(buf('t', [2, 3, 4], 'f32'), [idx('i'), idx('j'), idx('k')]), 'i * 12 + j * 4 + k');
    assert.strictEqual(fi(buf('m', [3, 4], 'f32'), [I(0), idx('j')]), 'j');
    assert.strictEqual(fi(buf('m', [3, 4], 'f32'), [I(0), I(0)]), '0');
  });

  // runPlan checks every step's arguments before it touches the device: an
  // undersized or mistyped slot is a JS error here, where no device exists
  {
    const L = linearSet();
    const provider = hip.createHipProvider('external_codegen', 'const_buffers');
    const codegen = hip.createHipExternalCodegen('const_buffers');
    const kernelOf = (pf) => { provider.annotate([pf]); return codegen.compile(pf, hip.hipTarget(), pf.getAttr('external_codegen').info); };
    const S = (pf, ins, outs) => ({ name: pf.name, inputSlots: ins, outputSlots: outs, kernel: kernelOf(pf), shapeValues: null });
    const steps = [S(L.pf.quantize, [0], [2]), S(L.pf.qmatmul, [2], [3]), S(L.pf.fused, [3, 1], [4])];
    const plan = { numSlots: 5, argSlots: [0, 1, 4], intermediates: [],
                   steps: steps.map((x) => ({ name: x.name, inputSlots: x.inputSlots, outputSlots: x.outputSlots })) };
    const mk = (data) => ({ data, shape: [data.length], dtype: 'f32' });
    const good = () => [mk(new Float32Array(M * K)), mk(new Float32Array(N)), mk(new Int8Array(M * K)),
                        mk(new Int32Array(M * N)), mk(new Float32Array(M * N))];
    const be = hip.createHipRuntimeBackend();
    test('runPlan rejects an undersized plan argument before any device call', () => {
      const sl = good();
      sl[0] = mk(new Float32Array(M * K - 1));
      assert.throws(() => hip.runPlanSync(plan, sl, steps), /quantize input has \d+ elements, expected \d+/);
      const s2 = good();
      s2[4] = mk(new Float32Array(M * N - 3));
      assert.throws(() => hip.runPlanSync(plan, s2, steps), /out has \d+ elements, expected/);
      const s3 = good();
      s3[3] = mk(new Float32Array(M * N));                  // the int32 accumulator slot as f32
      assert.throws(() => hip.runPlanSync(plan, s3, steps), /must be a Int32Array/);
    });
    testAsync('runPlan (the promise form) rejects an undersized plan argument', () => {
      const sl = good();
      sl[1] = mk(new Float32Array(N - 1));
      return be.runPlan(plan, sl, steps).then(() => { throw new Error('runPlan resolved'); },
                                              (e) => assert.ok(/has \d+ elements, expected/.test(e.message), e.message));
    });
  }

  test('the oracle per-channel tail agrees with q8ref.js (two restatements, one engine)', () => {
    const L = linearSet();
    const accD = randI32(7, M * N, 1 << 22), bD = normal(8, N, 0.1);
    const y1 = new Float32Array(M * N), y2 = new Float32Array(M * N);
    q8ref.buildEpiloguePerChannel(M, N, false, false)(accD, L.consts.sv.data, null, y1);
    ref.compilePrimFunc(L.pf.tail).fn(accD, y2, L.consts.sv.data);
    sameBits(y2, y1, 'tail');
    const z1 = new Float32Array(M * N), z2 = new Float32Array(M * N);
    q8ref.buildEpiloguePerChannel(M, N, true, true)(accD, L.consts.sv.data, bD, z1);
    ref.compilePrimFunc(L.pf.fused).fn(accD, bD, z2, L.consts.sv.data, L.consts.zero.data);
    sameBits(z2, z1, 'tail + bias + relu');
  });

  test('program layout matches the addon (sizeof q8_ew_prog)', () => {
    const a = require(path.join(ROOT, 'mlfw_amd', 'node', 'index.js'));
    assert.strictEqual(a.ewiseProgBytes(), ew.LAYOUT.bytes);
  });

  test('translated programs evaluate like the oracle (JS emulation of the device program)', () => {
    const L = linearSet();
    const { cases } = extraCases();
    const all = Object.entries(L.pf).filter(([k]) => k !== 'qmatmul').map(([k, pf]) => [k, pf]).concat(cases);
    let seed = 100;
    for (const [name, pf] of all) {
      const tr = ew.translateEwise(pf);
      assert.ok(tr, `${name}: not translated`);
      const consts = pf.getAttr('const_buffers') || [];
      const fill = (b) => {
        const c = consts.find((x) => x.buffer === b);
        if (c) return c.data;
        const a = alloc(b);
        if (a instanceof Float32Array) { a.set(withEdges(normal(seed++, a.length, 3))); }
        else if (a instanceof Int32Array) a.set(randI32(seed++, a.length, 1 << 26));
        else if (a instanceof Int8Array) a.set(randI8(seed++, a.length));
        return a;
      };
      const args = argsFor(pf, fill);
      const want = args.slice(), got = args.slice();
      want[tr.outIdx] = alloc(pf.bufferMap.get([...pf.bufferMap.keys()][tr.outIdx]));
      got[tr.outIdx] = alloc(pf.bufferMap.get([...pf.bufferMap.keys()][tr.outIdx]));
      ref.compilePrimFunc(pf).fn(...want);
      emulate(tr, got);
      sameBits(got[tr.outIdx], want[tr.outIdx], name);
    }
  });

  test('matchEpilogue finds the per-channel tail, bias, ReLU and requant forms only', () => {
    const L = linearSet();
    const zeroParam = (pf) => (p) => [...pf.bufferMap.values()][p] === L.bufs.zero;
    const m = (pf) => ew.matchEpilogue(ew.translateEwise(pf), zeroParam(pf));
    const t = m(L.pf.tail);
    assert.ok(t && !t.relu && t.biasParam < 0 && !t.quant && t.M === M && t.N === N);
    const f = m(L.pf.fused);
    assert.ok(f && f.relu && f.biasParam >= 0 && !f.quant);
    const r = m(L.pf.fusedRq);
    assert.ok(r && r.relu && r.quant && r.quant.scale === 0.0371);
    assert.strictEqual(m(L.pf.add), null);
    assert.strictEqual(m(L.pf.reluQuant), null);
    const { cases } = extraCases();
    for (const [, pf] of cases) assert.strictEqual(ew.matchEpilogue(ew.translateEwise(pf), () => false), null);
  });

  test('the provider tags every PrimFunc of the linear set; nothing reaches the host codegen', () => {
    const L = linearSet();
    const p = hip.createHipProvider('external_codegen', 'const_buffers');
    const pfs = Object.values(L.pf);
    p.annotate(pfs);
    for (const pf of pfs) {
      const a = pf.getAttr('external_codegen');
      assert.ok(a && a.name === 'hip_int8', `${pf.name} untagged`);
    }
    assert.strictEqual(L.pf.qmatmul.getAttr('external_codegen').info.op, 'quantized_dot');
    assert.strictEqual(L.pf.quantize.getAttr('external_codegen').info.op, 'quantize');
    assert.ok(L.pf.fused.getAttr('external_codegen').info.epilogue.relu);
  });

  test('BackendPipeline.compile with the hip entries: tagged -> hip kernels, the rest -> host codegen', () => {
    // restates src/backend/pipeline.ts:37-57
    const externals = new Map(), entries = new Map();
    entries.set('cpu', { runtimeKind: 'js', compile: (pf) => ({ source: `function ${pf.name}(){}`, metadata: { kind: 'js' } }) });
    const r = { registerBackend() {}, registerExternalCodegen: (n, e) => externals.set(n, e),
                registerExternalCodegenProvider() {}, registerCodegen: (k, e) => entries.set(k, e),
                getCodegenEntry: (k) => entries.get(k) || null, FuncAttr: { EXTERNAL_CODEGEN: 'external_codegen', CONST_BUFFERS: 'const_buffers' } };
    hip.registerHip(r);
    const target = hip.hipTarget();
    function compile(pf) {
      const x = pf.getAttr('external_codegen');
      if (x) {
        const e = externals.get(x.name);
        if (e && e.targetKind === target.kind) return e.compile(pf, target, x.info);
      }
      const entry = r.getCodegenEntry(target.kind);
      if (!entry) throw new Error(`Unsupported target kind: ${target.kind}`);
      return entry.compile(pf, target);
    }
    const L = linearSet();
    hip.createHipProvider('external_codegen', 'const_buffers').annotate(Object.values(L.pf));
    for (const pf of Object.values(L.pf)) {
      const k = compile(pf);
      assert.strictEqual(k.metadata.kind, 'hip', pf.name);
    }
    const qk = compile(L.pf.qmatmul);
    assert.ok(qk.metadata.constBuffers && qk.metadata.constBuffers[0].data === L.consts.W.data, 'const buffers travel');
    // a reduction (not an elementwise nest): compiled for the host, labelled
    const s = buf('s', [M], 'f32'), x = buf('x', [M, K], 'f32');
    const red = primFunc('sum', [x, s], { type: 'ForNode', loopVar: V('r0'), min: I(0), extent: I(M), kind: 'serial',
      body: { type: 'BlockNode', name: 'reduce', iterVars: [], reads: [], writes: [], initBody: { type: 'SeqNode', stmts: [] },
              body: { type: 'BufferStoreNode', buffer: s, indices: [V('r0')], value: F(0) } } });
    hip.createHipProvider('external_codegen', 'const_buffers').annotate([red]);
    const rk = compile(red);
    assert.strictEqual(rk.metadata.kind, 'js');
    assert.strictEqual(rk.metadata.hipRoute, 'host');
  });

  test('q8 activation mode travels on the target into the quantize descriptors', () => {
    assert.strictEqual(hip.activationMode(hip.hipTarget()), 'static');
    const t = hip.hipTarget(null, null, { activations: 'per_token' });
    assert.strictEqual(t.getAttr(hip.ACTIVATIONS_ATTR), 'per_token');
    assert.throws(() => hip.hipTarget(null, null, { activations: 'per_row' }), /q8 activations must be one of/);
    // with the reference factory: TargetFeatures.withAttr (support/target.ts:145-147)
    const made = hip.hipTarget((cfg) => {
      const attrs = new Map();
      return Object.assign({}, cfg, { getAttr: (k, f = null) => (attrs.has(k) ? attrs.get(k) : f),
                                      withAttr(k, v) { attrs.set(k, v); return this; } });
    }, null, { activations: 'per_tensor' });
    assert.strictEqual(hip.activationMode(made), 'per_tensor');
    const L = linearSet();
    const cg = hip.createHipExternalCodegen('const_buffers');
    const prov = hip.createHipProvider('external_codegen', 'const_buffers');
    prov.annotate([L.pf.quantize, L.pf.qmatmul]);
    const kq = cg.compile(L.pf.quantize, t, L.pf.quantize.getAttr('external_codegen').info);
    const kd = cg.compile(L.pf.qmatmul, t, L.pf.qmatmul.getAttr('external_codegen').info);
    assert.strictEqual(kq.metadata.q8.activations, 'per_token');
    assert.strictEqual(kd.metadata.q8.activations, undefined);
    const ks = cg.compile(L.pf.quantize, hip.hipTarget(), L.pf.quantize.getAttr('external_codegen').info);
    assert.strictEqual(ks.metadata.q8.activations, undefined);
  });

  test('hipTarget builds on the reference factory when given one', () => {
    const seen = [];
    const t = hip.hipTarget((cfg) => { seen.push(cfg); return { kind: cfg.kind, made: true }; });
    assert.ok(t.made);
    assert.strictEqual(seen[0].kind, 'hip');
    assert.strictEqual(seen[0].supportsInt8, true);
    assert.strictEqual(hip.hipTarget().isGPU(), false);
  });
}

// ---------------------------------------------------------------- GPU tests
/** RuntimeModule.runPlanAsync (runtime.ts:290-329) for a uniform plan. */
function makePlan(steps, argSlots, numSlots) {
  return { numSlots, argSlots, intermediates: [], steps: steps.map((s) => ({ name: s.name, inputSlots: s.inputSlots,
                                                                           outputSlots: s.outputSlots })) };
}

function gpuTests() {
  const A = require(path.join(ROOT, 'mlfw_amd', 'node', 'index.js'));
  A.init(0);
  const codegen = hip.createHipExternalCodegen('const_buffers');
  const provider = hip.createHipProvider('external_codegen', 'const_buffers');
  const be = hip.createHipRuntimeBackend();
  const kernelOf = (pf) => {
    provider.annotate([pf]);
    const x = pf.getAttr('external_codegen');
    assert.ok(x, `${pf.name} not tagged`);
    return codegen.compile(pf, hip.hipTarget(), x.info);
  };
  // RuntimeModule.run: tensor args + const buffers appended (runtime.ts:246-268)
  const runKernel = (kernel, inst, args) => {
    const all = args.concat((kernel.metadata.constBuffers || []).map((c) => c.data));
    be.runSync(inst, all, null);
  };

  test('GPU: every elementwise PrimFunc through runSync, bit for bit', () => {
    const L = linearSet();
    const { cases } = extraCases();
    const all = Object.entries(L.pf).filter(([k]) => k !== 'qmatmul').concat(cases);
    let seed = 300;
    for (const [name, pf] of all) {
      const consts = pf.getAttr('const_buffers') || [];
      const fill = (b) => {
        const c = consts.find((x) => x.buffer === b);
        if (c) return c.data;
        const a = alloc(b);
        if (a instanceof Float32Array) a.set(withEdges(normal(seed++, a.length, 3)));
        else if (a instanceof Int32Array) a.set(randI32(seed++, a.length, 1 << 26));
        else if (a instanceof Int8Array) a.set(randI8(seed++, a.length));
        return a;
      };
      const args = argsFor(pf, fill);
      const kernel = kernelOf(pf);
      const d = kernel.metadata.q8;
      const outIdx = d.outIdx;
      const want = args.slice();
      want[outIdx] = alloc([...pf.bufferMap.values()][outIdx]);
      ref.compilePrimFunc(pf).fn(...want);
      const nParams = [...pf.bufferMap.values()].length - consts.length;
      const got = args.slice(0, nParams);
      got[outIdx] = alloc([...pf.bufferMap.values()][outIdx]);
      runKernel(kernel, be.instantiate(kernel), got);
      sameBits(got[outIdx], want[outIdx], name);
    }
  });

  // the whole per-channel Linear + bias + ReLU set, layer output requantized
  function linearRun(which, fuse) {
    const L = linearSet();
    const xD = withEdges(normal(21, M * K, 1.5)), bD = normal(22, N, 0.05);
    // oracle: every step on the host
    const h = {};
    const run = (pf, args) => ref.compilePrimFunc(pf).fn(...args);
    h.xq = new Int8Array(M * K); run(L.pf.quantize, [xD, h.xq]);
    h.acc = new Int32Array(M * N); q8ref.buildQuantizedDot(M, N, K, 1, 0, 0)(h.xq, L.consts.W.data, h.acc);
    const sv = L.consts.sv.data, zero = L.consts.zero.data;
    h.y = new Float32Array(M * N); run(L.pf.tail, [h.acc, h.y, sv]);
    h.y2 = new Float32Array(M * N); run(L.pf.add, [h.y, bD, h.y2]);
    h.y3 = new Float32Array(M * N); run(L.pf.max, [h.y2, h.y3, zero]);
    h.q2 = new Int8Array(M * N); run(L.pf.reluQuant, [h.y2, h.q2, zero]);
    // slots: 0 x, 1 b, 2 xq, 3 acc, 4 y, 5 y2, 6 y3 / q2
    let steps, outSlot, want;
    const S = (pf, ins, outs) => ({ name: pf.name, inputSlots: ins, outputSlots: outs, kernel: kernelOf(pf), shapeValues: null });
    if (which === 'unfused') {
      steps = [S(L.pf.quantize, [0], [2]), S(L.pf.qmatmul, [2], [3]), S(L.pf.tail, [3], [4]),
               S(L.pf.add, [4, 1], [5]), S(L.pf.max, [5], [6])];
      outSlot = 6; want = h.y3;
    } else if (which === 'fused') {
      steps = [S(L.pf.quantize, [0], [2]), S(L.pf.qmatmul, [2], [3]), S(L.pf.fused, [3, 1], [6])];
      outSlot = 6; want = h.y3;
    } else {
      steps = [S(L.pf.quantize, [0], [2]), S(L.pf.qmatmul, [2], [3]), S(L.pf.fusedRq, [3, 1], [6])];
      outSlot = 6; want = h.q2;
    }
    const plan = makePlan(steps, [0, 1, outSlot], 7);
    const mk = (data, shape, dtype) => ({ data, shape, dtype });
    const out = which === 'requant' ? new Int8Array(M * N) : new Float32Array(M * N);
    const slots = [mk(xD, [M, K], 'f32'), mk(bD, [N], 'f32'), mk(new Int8Array(M * K), [M, K], 'i8'),
                   mk(new Int32Array(M * N), [M, N], 'i32'), mk(new Float32Array(M * N), [M, N], 'f32'),
                   mk(new Float32Array(M * N), [M, N], 'f32'), mk(out, [M, N], which === 'requant' ? 'i8' : 'f32')];
    return { plan, slots, steps, out, want, h, fuse, L, xD, bD };
  }

  // the oracle of linearRun's plans for any input x (host, step by step)
  function oracleLinear(L, which, xD, bD) {
    const run = (pf, args) => ref.compilePrimFunc(pf).fn(...args);
    const xq = new Int8Array(M * K); run(L.pf.quantize, [xD, xq]);
    const acc = new Int32Array(M * N); q8ref.buildQuantizedDot(M, N, K, 1, 0, 0)(xq, L.consts.W.data, acc);
    const y = new Float32Array(M * N); run(L.pf.tail, [acc, y, L.consts.sv.data]);
    const y2 = new Float32Array(M * N); run(L.pf.add, [y, bD, y2]);
    if (which === 'requant') { const q2 = new Int8Array(M * N); run(L.pf.reluQuant, [y2, q2, L.consts.zero.data]); return q2; }
    const y3 = new Float32Array(M * N); run(L.pf.max, [y2, y3, L.consts.zero.data]);
    return y3;
  }

  test('GPU: resident plan inputs are not uploaded again while their key and version are unchanged', () => {
    const t = linearRun('fused', true);
    t.slots[0].resident = { key: t.slots[0].data, version: 1 };
    t.slots[1].resident = { key: t.slots[1].data, version: 1 };
    hip.resetStats();
    hip.runPlanSync(t.plan, t.slots, t.steps, { resident: true });
    sameBits(t.out, t.want, 'first call');
    assert.strictEqual(hip.stats.uploadBytes - hip.stats.constUploadBytes, 4 * M * K + 4 * N, 'first call uploads x and b');
    hip.resetStats();
    t.out.fill(0);
    hip.runPlanSync(t.plan, t.slots, t.steps, { resident: true });
    sameBits(t.out, t.want, 'second call');
    assert.strictEqual(hip.stats.uploadBytes, 0, 'second call with unchanged arguments uploads 0 bytes');
    assert.strictEqual(hip.stats.residentSkips, 2);
    // a new version of x is uploaded, b stays
    const x2 = normal(77, M * K, 1.5);
    t.slots[0].data.set(x2);
    t.slots[0].resident.version = 2;
    hip.resetStats();
    hip.runPlanSync(t.plan, t.slots, t.steps, { resident: true });
    assert.strictEqual(hip.stats.uploadBytes, 4 * M * K, 'only the new version of x');
    sameBits(t.out, oracleLinear(t.L, 'fused', x2, t.bD), 'new x');
    // without {resident: true} every input is uploaded
    hip.resetStats();
    hip.runPlanSync(t.plan, t.slots, t.steps);
    assert.strictEqual(hip.stats.uploadBytes, 4 * M * K + 4 * N);
  });

  test('GPU: slots share device buffers by the plan buffer assignment', () => {
    const t = linearRun('unfused', false);
    // slots: 0 x, 1 b, 2 xq, 3 acc, 4 y, 5 y2, 6 y3: xq / y and acc / y2 do not overlap in time
    t.plan.buffers = { slotBuffer: [0, 1, 2, 3, 2, 3, 4], bufferBytes: [4 * M * K, 4 * N, 4 * M * N, 4 * M * N, 4 * M * N] };
    for (let c = 0; c < 2; c++) {
      t.out.fill(0);
      hip.runPlanSync(t.plan, t.slots, t.steps, { fuse: false });
      sameBits(t.out, t.want, `grouped slots, call ${c}`);
    }
    hip.releasePlan(t.plan);
  });

  testAsync('GPU: runPlan (the promise form) downloads when the device has finished, queues overlapping calls on one plan', () => {
    const be = hip.createHipRuntimeBackend();
    const t = linearRun('fused', true);
    // a second call on the same plan (the same device buffers) with another
    // x and its own output, made before the first has settled
    const x2 = normal(91, M * K, 1.5);
    const out2 = new Float32Array(M * N);
    const slots2 = t.slots.map((sl, i) => ({ ...sl, data: i === 0 ? x2 : i === 6 ? out2 : sl.data.slice() }));
    const p1 = be.runPlan(t.plan, t.slots, t.steps);
    assert.ok(p1 instanceof Promise);
    assert.ok(t.out.every((v) => v === 0), 'the output is downloaded when the promise settles, not before');
    assert.throws(() => hip.runPlanSync(t.plan, t.slots, t.steps), /still in flight/);
    assert.throws(() => hip.releasePlan(t.plan), /still in flight/);
    const p2 = be.runPlan(t.plan, slots2, t.steps);
    return Promise.all([p1, p2]).then(() => {
      sameBits(t.out, t.want, 'first call');
      sameBits(out2, oracleLinear(t.L, 'fused', x2, t.bD), 'second call, queued behind the first');
      hip.runPlanSync(t.plan, t.slots, t.steps);             // settled: the plan runs synchronously again
      sameBits(t.out, t.want, 'runPlanSync after the promises');
      hip.releasePlan(t.plan);
    });
  });

  testAsync('GPU: runPlan (the promise form) in graph mode: eager, captured and replayed runs queue and match', () => {
    const be = hip.createHipRuntimeBackend();
    const t = linearRun('fused', true);
    const xs = [normal(101, M * K, 1.5), normal(102, M * K, 1.5), normal(103, M * K, 1.5), normal(104, M * K, 1.5)];
    const outs = xs.map(() => new Float32Array(M * N));
    const runs = xs.map((x, i) => be.runPlan(t.plan, t.slots.map((sl, j) => ({ ...sl, data: j === 0 ? x : j === 6 ? outs[i] : sl.data.slice() })),
                                             t.steps, { graph: true }));
    return Promise.all(runs).then(() => {
      xs.forEach((x, i) => sameBits(outs[i], oracleLinear(t.L, 'fused', x, t.bD), `graph-mode run ${i}`));
      hip.releasePlan(t.plan);
    });
  });

  for (const [which, fuse] of [['fused', true], ['unfused', false], ['requant', true]]) {
    test(`GPU: runPlan in graph mode (${which}, fusion ${fuse ? 'on' : 'off'}): eager, captured, replayed, fresh x every call`, () => {
      const t = linearRun(which, fuse);
      const A = require(path.join(ROOT, 'mlfw_amd', 'node', 'index.js'));
      hip.resetStats();
      for (let c = 0; c < 5; c++) {
        const x = normal(90 + c, M * K, 1.5);
        t.slots[0].data.set(x);
        t.out.fill(0);
        hip.runPlanSync(t.plan, t.slots, t.steps, { graph: true, fuse });
        sameBits(t.out, oracleLinear(t.L, which, x, t.bD), `${which} call ${c}`);
        // eager device work and a synchronization between replays
        const junk = A.alloc(4096);
        A.fillUniform(junk, 1024, 5, 0, 0, 1);
        A.sync();
        A.free(junk);
      }
      assert.strictEqual(hip.stats.graphCaptures, 1, 'captured once (on the second call)');
      assert.strictEqual(hip.stats.graphReplays, 4, 'calls 2-5 replay');
      // a constant marked dirty drops the graph: one eager call, then a new capture
      hip.markHostDirty(t.L.consts.W.data);
      for (let c = 0; c < 3; c++) {
        t.out.fill(0);
        hip.runPlanSync(t.plan, t.slots, t.steps, { graph: true, fuse });
        sameBits(t.out, oracleLinear(t.L, which, t.slots[0].data, t.bD), `${which} after markHostDirty, call ${c}`);
      }
      assert.strictEqual(hip.stats.graphCaptures, 2);
      hip.releasePlan(t.plan);
    });
  }

  test('GPU: the addon rejects device buffers smaller than the call needs', () => {
    const A = require(path.join(ROOT, 'mlfw_amd', 'node', 'index.js'));
    const small = A.alloc(16), big = A.alloc(64 * 64 * 4);
    assert.throws(() => A.gemm(small, big, 64, 64, 64, 0, 0, null, 0, null, 0, A.Q8_EPI_PT, 1.0, null, 0, A.Q8_I32, big),
                  /gemm A device buffer holds 16 bytes, the call needs 4096/);
    assert.throws(() => A.gemm(big, big, 64, 64, 64, 0, 0, null, 0, null, 0, A.Q8_EPI_PT, 1.0, null, 0, A.Q8_I32, small),
                  /gemm out device buffer holds 16 bytes, the call needs 16384/);
    assert.throws(() => A.quantizeRows(big, 64, 64, A.Q8_PER_TOKEN, big, small), /quantizeRows scales/);
    assert.throws(() => A.dequantize(small, A.Q8_I32, 2, 4, big, A.Q8_PER_TENSOR, 0, big), /dequantize q/);
    assert.throws(() => A.fillNormal(small, 5, 1, 0, 0, 1), /fill output/);
    A.free(small);
    A.free(big);
  });


  for (const [which, fuse, fusedCount] of [['unfused', true, 1], ['unfused', false, 0], ['fused', true, 1],
                                            ['fused', false, 0], ['requant', true, 1], ['requant', false, 0]]) {
    test(`GPU: runPlan of the per-channel linear set (${which}, fusion ${fuse ? 'on' : 'off'})`, () => {
      const t = linearRun(which, fuse);
      hip.resetStats();
      let err = null;
      try { hip.runPlanSync(t.plan, t.slots, t.steps, { fuse }); } catch (e) { err = e; }
      const first = Object.assign({}, hip.stats);
      sameBits(t.out, t.want, `${which} plan output`);
      assert.strictEqual(first.fusedLinears, fusedCount);
      // intermediates stay on the device: only plan outputs come back
      assert.strictEqual(t.slots[3].data.some((v) => v !== 0), false, 'acc slot was never downloaded');
      // a second run uploads no constant bytes and only the plan inputs
      hip.resetStats();
      t.out.fill(0);
      try { hip.runPlanSync(t.plan, t.slots, t.steps, { fuse }); } catch (e) { err = e; }
      assert.strictEqual(err, null);
      sameBits(t.out, t.want, `${which} plan output, second run`);
      assert.strictEqual(hip.stats.constUploadBytes, 0, 'weights uploaded again');
      assert.strictEqual(hip.stats.uploadBytes, 4 * M * K + 4 * N, 'second run uploads only x and b');
    });
  }

  // per-token / per-tensor dynamic activations (hipTarget q8 activations)
  const S = (pf, ins, outs, target) => ({ name: pf.name, inputSlots: ins, outputSlots: outs, shapeValues: null,
                                           kernel: (() => { provider.annotate([pf]);
                                             return codegen.compile(pf, target || hip.hipTarget(), pf.getAttr('external_codegen').info); })() });
  const mkSlot = (data, shape, dtype) => ({ data, shape, dtype });
  function dynamicWant(L, x, b, mode) {
    // the oracle of the dynamic form: S-token (or S-abs over the tensor), R1,
    // quantized_dot, then fround(acc * fround(sx[m] * (sv[n] / s))) + bias, ReLU
    const sx = new Float64Array(M);
    if (mode === 'per_tensor') { const t = q8ref.scalesPerToken(x, 1, M * K, new Float64Array(1)); sx.fill(t[0]); }
    else q8ref.scalesPerToken(x, M, K, sx);
    const xq = new Int8Array(M * K); q8ref.buildQuantizeRows(M, K)(x, sx, xq);
    const acc = new Int32Array(M * N); q8ref.buildQuantizedDot(M, N, K, 1, 0, 0)(xq, L.consts.W.data, acc);
    const sv = L.consts.sv.data, y = new Float32Array(M * N);
    for (let m = 0; m < M; m++) for (let n = 0; n < N; n++) {
      const v = Math.fround(Math.fround((+acc[m * N + n]) * Math.fround(sx[m] * (sv[n] / L.sX))) + b[n]);
      y[m * N + n] = Math.max(v, 0);
    }
    return y;
  }
  for (const mode of ['per_token', 'per_tensor']) {
    test(`GPU: runPlan with ${mode} dynamic activations: one q8_qlinear_dynamic launch, bit for bit`, () => {
      const L = linearSet();
      const x = normal(31, M * K, 1.5), b = normal(32, N, 0.05);
      for (let k = 0; k < K; k++) x[3 * K + k] = 0;            // a row of zeros: scale 1e-10
      const tq = hip.hipTarget(null, null, { activations: mode });
      const steps = [S(L.pf.quantize, [0], [2], tq), S(L.pf.qmatmul, [2], [3]), S(L.pf.fused, [3, 1], [4])];
      const plan = makePlan(steps, [0, 1, 4], 5);
      const out = new Float32Array(M * N);
      const slots = [mkSlot(x, [M, K], 'f32'), mkSlot(b, [N], 'f32'), mkSlot(new Int8Array(M * K), [M, K], 'i8'),
                     mkSlot(new Int32Array(M * N), [M, N], 'i32'), mkSlot(out, [M, N], 'f32')];
      hip.resetStats();
      let err = null;
      try { hip.runPlanSync(plan, slots, steps); } catch (e) { err = e; }
      assert.strictEqual(err, null);
      assert.strictEqual(hip.stats.launches, 1, 'one launch for the linear');
      assert.strictEqual(hip.stats.dynamicLinears, 1);
      sameBits(out, dynamicWant(L, x, b, mode), `${mode} dynamic linear`);
      // the run-time option overrides the compiled mode, and 'static' is the reference's result
      const stat = new Float32Array(M * N);
      slots[4] = mkSlot(stat, [M, N], 'f32');
      try { hip.runPlanSync(plan, slots, steps, { q8Activations: 'static' }); } catch (e) { err = e; }
      assert.strictEqual(err, null);
      const h = {};
      h.xq = new Int8Array(M * K); ref.compilePrimFunc(L.pf.quantize).fn(x, h.xq);
      h.acc = new Int32Array(M * N); q8ref.buildQuantizedDot(M, N, K, 1, 0, 0)(h.xq, L.consts.W.data, h.acc);
      h.y = new Float32Array(M * N); ref.compilePrimFunc(L.pf.fused).fn(h.acc, b, h.y, L.consts.sv.data, L.consts.zero.data);
      sameBits(stat, h.y, 'static plan');
    });
  }

  test('GPU: a dynamic scale equal to the static one gives the static result', () => {
    const sX = 4.5 / 127;                    // 4.5 is a float: the per-tensor absmax below
    const L = linearSet(sX);
    const x = normal(33, M * K, 1.0), b = normal(34, N, 0.05);
    for (let i = 0; i < x.length; i++) x[i] = Math.max(-4.25, Math.min(4.25, x[i]));
    x[17] = -4.5;
    const run = (target) => {
      const steps = [S(L.pf.quantize, [0], [2], target), S(L.pf.qmatmul, [2], [3]), S(L.pf.fused, [3, 1], [4])];
      const out = new Float32Array(M * N);
      const slots = [mkSlot(x, [M, K], 'f32'), mkSlot(b, [N], 'f32'), mkSlot(new Int8Array(M * K), [M, K], 'i8'),
                     mkSlot(new Int32Array(M * N), [M, N], 'i32'), mkSlot(out, [M, N], 'f32')];
      let err = null;
      try { hip.runPlanSync(makePlan(steps, [0, 1, 4], 5), slots, steps); } catch (e) { err = e; }
      assert.strictEqual(err, null);
      return out;
    };
    hip.resetStats();
    const dyn = run(hip.hipTarget(null, null, { activations: 'per_tensor' }));
    assert.strictEqual(hip.stats.dynamicLinears, 1);
    sameBits(dyn, run(hip.hipTarget()), 'per-tensor dynamic vs static');
  });

  test('GPU: three linears, each layer requantized in its GEMM epilogue: one launch per linear', () => {
    // x -> quantize -> [qmatmul, fused relu+requant] -> [qmatmul, fused relu+requant] -> [qmatmul, tail]
    // (every layer [N,K] = [K,K] so the layers chain), against the oracle run step by step
    const Kx = K;
    // layer i reads the previous layer's int8 codes: the quantize scale of
    // layer i+1 is the sNext the fused requant of layer i writes with
    const layers = [];
    for (let i = 0; i < 3; i++) {
      const xq = buf(`xq${i}`, [M, Kx], 'i8'), W = buf(`w${i}`, [Kx, Kx], 'i8'), acc = buf(`acc${i}`, [M, Kx], 'i32');
      const sv = buf(`sv${i}`, [Kx], 'f32'), b = buf(`b${i}`, [Kx], 'f32'), zero = buf(`zero${i}`, [1, 1], 'f32');
      const out = buf(`o${i}`, [M, Kx], i < 2 ? 'i8' : 'f32');
      const sIn = i === 0 ? 4.9 / 127 : 0.0371 * (1 + i);
      const sOut = 0.0371 * (2 + i);
      const Wd = randI8(50 + i, Kx * Kx), svd = new Float32Array(Kx);
      for (let n = 0; n < Kx; n++) svd[n] = Math.fround(sIn * (0.001 + 0.0002 * ((n * 31 + i) % 13)));
      const cW = { buffer: W, data: Wd }, cS = { buffer: sv, data: svd }, cZ = { buffer: zero, data: new Float32Array([0]) };
      const body = (l) => ext('max', [math('+', math('*', cast(l[0], 'i32', 'f32'), l[1]), l[2]), l[3]]);
      layers.push({
        qmm: qmatmulPF(M, Kx, Kx, xq, W, acc, [cW]),
        epi: i < 2 ? pointwise(`fused_rq${i}`, out, [acc, sv, b, zero], (l) => quantizeExpr(body(l), sOut), [cS, cZ])
                   : pointwise(`fused_tail${i}`, out, [acc, sv, b, zero], body, [cS, cZ]),
        W: Wd, sv: svd, sOut,
      });
    }
    const x0 = buf('x0', [M, Kx], 'f32'), q0 = buf('q0', [M, Kx], 'i8');
    const quant0 = pointwise('quantize0', q0, [x0], (l) => quantizeExpr(l[0], 4.9 / 127));
    const x = withEdges(normal(40, M * Kx, 1.5));
    const bs = [normal(41, Kx, 0.05), normal(42, Kx, 0.05), normal(43, Kx, 0.05)];
    // slots: 0 x, 1..3 biases, 4 q0, 5 acc0, 6 q1, 7 acc1, 8 q2, 9 acc2, 10 y
    const steps = [S(quant0, [0], [4])];
    for (let i = 0; i < 3; i++) {
      steps.push(S(layers[i].qmm, [4 + 2 * i], [5 + 2 * i]));
      steps.push(S(layers[i].epi, [5 + 2 * i, 1 + i], [i < 2 ? 6 + 2 * i : 10]));
    }
    const y = new Float32Array(M * Kx);
    const slots = [mkSlot(x, [M, Kx], 'f32'), mkSlot(bs[0], [Kx], 'f32'), mkSlot(bs[1], [Kx], 'f32'), mkSlot(bs[2], [Kx], 'f32')];
    for (let i = 0; i < 3; i++) {
      slots.push(mkSlot(new Int8Array(M * Kx), [M, Kx], 'i8'));
      slots.push(mkSlot(new Int32Array(M * Kx), [M, Kx], 'i32'));
    }
    slots.push(mkSlot(y, [M, Kx], 'f32'));
    // oracle, step by step on the host
    let cur = new Int8Array(M * Kx);
    ref.compilePrimFunc(quant0).fn(x, cur);
    let want = null;
    for (let i = 0; i < 3; i++) {
      const acc = new Int32Array(M * Kx);
      q8ref.buildQuantizedDot(M, Kx, Kx, 1, 0, 0)(cur, layers[i].W, acc);
      const o = i < 2 ? new Int8Array(M * Kx) : new Float32Array(M * Kx);
      ref.compilePrimFunc(layers[i].epi).fn(acc, bs[i], o, layers[i].sv, new Float32Array([0]));  // params: acc, b, out, sv, zero
      if (i < 2) cur = o; else want = o;
    }
    hip.resetStats();
    let err = null;
    try { hip.runPlanSync(makePlan(steps, [0, 1, 2, 3, 10], 11), slots, steps); } catch (e) { err = e; }
    assert.strictEqual(err, null);
    sameBits(y, want, 'three-layer output');
    assert.strictEqual(hip.stats.fusedLinears, 3);
    assert.strictEqual(hip.stats.launches, 4, 'the input quantize + one GEMM per linear');
  });

  test('GPU: runSync of the linear set step by step, weights resident after the first call', () => {
    const t = linearRun('unfused', true);
    const insts = t.steps.map((s) => be.instantiate(s.kernel));
    const host = (slot) => t.slots[slot].data;
    const once = () => t.steps.forEach((s, k) => runKernel(s.kernel, insts[k], s.inputSlots.concat(s.outputSlots).map(host)));
    hip.resetStats();
    once();
    sameBits(host(3), t.h.acc, 'acc');
    sameBits(host(6), t.want, 'y3');
    assert.ok(hip.stats.constUploadBytes >= N * K, 'the int8 weight was uploaded once');
    hip.resetStats();
    once();
    assert.strictEqual(hip.stats.constUploadBytes, 0, 'second call uploads no weight bytes');
    sameBits(host(6), t.want, 'y3, second call');
  });
}

const mode = process.argv[2] || 'cpu';
if (mode === 'cpu') cpuTests();
else gpuTests();
Promise.all(pending).then(() => {
  console.log(failures ? `${failures} failed` : 'all passed');
  process.exit(failures ? 1 : 0);
});
