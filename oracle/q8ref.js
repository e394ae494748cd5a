'use strict';
/*
 * q8ref.js -- JavaScript mirror of the kernels mlfw's CPU backend generates
 * for the int8 path.  TEST INFRASTRUCTURE ONLY (cross-check of the C oracle
 * against a real JS engine, and the timed single-thread CPU baseline).
 *
 * The reference's CPU backend emits one plain `function` per fused group and
 * instantiates it with `new Function` (src/backend/cpu/codegen.ts:65-146,
 * src/runtime/backend_registry.ts:141-154).  The builders below emit source
 * text of the same shape with the same expression forms:
 *   quantize   (quant_math.ts:16-27, codegen.ts:496,519,534):
 *     q[i] = (Math.min(Math.max(Math.round(Math.fround(x[i] / S)), -128), 127) | 0);
 *   dequantize (quant_math.ts:29-34):  y[i] = Math.fround((+q[i]) * S);
 *   quantized_dot (rules/quantization.ts:57-76, codegen.ts:257-275): zero-init
 *     nest, then a k loop on a local `_acc_1` that is stored once;
 *   per-channel epilogue (quantization_pass.ts:431-456): convert+broadcast+mul
 *     fused:  y[i] = Math.fround((+acc[i]) * sv[n])  with sv a Float32Array.
 * Scalars are printed with String(v) (FloatImmNode, codegen.ts:441), which
 * round-trips every double exactly.
 *
 * Node v12 compatible (CommonJS, no optional chaining).
 */

const fs = require('fs');

// ---- src/util/random.ts:5-14 ------------------------------------------
function makeRng(seed) {
  let a = seed >>> 0;
  return function next() {
    a |= 0;
    a = (a + 0x6d2b79f5) | 0;
    let t = Math.imul(a ^ (a >>> 15), 1 | a);
    t = (t + Math.imul(t ^ (t >>> 7), 61 | t)) ^ t;
    return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
  };
}

// ---- src/nn/init.ts:40-52 (normal_) and :31-37 (uniform_) -------------
function normalFill(rng, out, mean, std) {
  for (let i = 0; i < out.length; i += 2) {
    const u1 = rng() || 1e-10;
    const u2 = rng();
    const r = Math.sqrt(-2 * Math.log(u1));
    const theta = 6.283185307179586 * u2;
    out[i] = mean + std * r * Math.cos(theta);
    if (i + 1 < out.length) out[i + 1] = mean + std * r * Math.sin(theta);
  }
  return out;
}

function uniformFill(rng, out, a, b) {
  const range = b - a;
  for (let i = 0; i < out.length; i++) out[i] = a + rng() * range;
  return out;
}

// ---- kernel builders (the generated-source shapes) ---------------------
function buildQuantize(n, scale, zeroPoint, unsigned) {
  const lo = unsigned ? 0 : -128, hi = unsigned ? 255 : 127;
  let scaled = `Math.fround(x[i] / ${String(scale)})`;
  if (zeroPoint !== 0) scaled = `Math.fround(${scaled} + ${String(zeroPoint)})`;
  const src = `for (let i = 0; i < ${n}; i++) {\n` +
    `  q[i] = (Math.min(Math.max(Math.round(${scaled}), ${lo}), ${hi}) | 0);\n}`;
  return new Function('x', 'q', src);
}

// Per-token quantize: the same expression with the row's scale read from a
// Float64Array (the value a per-row literal would print).
function buildQuantizeRows(M, K) {
  const src = `for (let m = 0; m < ${M}; m++) {\n` +
    `  const s = sc[m];\n` +
    `  for (let k = 0; k < ${K}; k++) {\n` +
    `    q[m * ${K} + k] = (Math.min(Math.max(Math.round(Math.fround(x[m * ${K} + k] / s)), -128), 127) | 0);\n` +
    `  }\n}`;
  return new Function('x', 'sc', 'q', src);
}

// Per-row dynamic scales: ValueObserver.update's min / max over the row
// (calibration.ts:24-34: plain < / > compares, so NaN never moves them),
// then fromRange symmetric (quantization_types.ts:249-253): absmax / 127,
// 0 or NaN -> 1e-10; an empty row keeps defaultForActivation's 6 / 127.
function scalesPerToken(x, M, K, out) {
  for (let m = 0; m < M; m++) {
    if (K === 0) { out[m] = 6 / 127; continue; }
    let lo = Infinity, hi = -Infinity;
    for (let k = 0; k < K; k++) {
      const v = x[m * K + k];
      if (v < lo) lo = v;
      if (v > hi) hi = v;
    }
    out[m] = Math.max(Math.abs(lo), Math.abs(hi)) / 127 || 1e-10;
  }
  return out;
}

function buildDequantize(n, scale, zeroPoint) {
  let v = '(+q[i])';
  if (zeroPoint !== 0) v = `Math.fround(${v} - ${String(zeroPoint)})`;
  const src = `for (let i = 0; i < ${n}; i++) {\n  y[i] = Math.fround(${v} * ${String(scale)});\n}`;
  return new Function('q', 'y', src);
}

function buildDequantizeRows(M, K) {
  const src = `for (let m = 0; m < ${M}; m++) {\n  const s = sc[m];\n` +
    `  for (let k = 0; k < ${K}; k++) {\n` +
    `    y[m * ${K} + k] = Math.fround((+q[m * ${K} + k]) * s);\n  }\n}`;
  return new Function('q', 'sc', 'y', src);
}

// bLayout 0: B is [K,N] (rhs_contracting=[0]); 1: B is [N,K] (=[1]).
function buildQuantizedDot(M, N, K, bLayout, zpA, zpB) {
  const bIdx = bLayout === 0 ? `k * ${N} + n` : `n * ${K} + k`;
  const a = zpA !== 0 ? `((A[m * ${K} + k] | 0) - ${zpA})` : `(A[m * ${K} + k] | 0)`;
  const b = zpB !== 0 ? `((B[${bIdx}] | 0) - ${zpB})` : `(B[${bIdx}] | 0)`;
  const src =
    `for (let m = 0; m < ${M}; m++) {\n  for (let n = 0; n < ${N}; n++) {\n` +
    `    out[m * ${N} + n] = 0;\n  }\n}\n` +
    `for (let m = 0; m < ${M}; m++) {\n  for (let n = 0; n < ${N}; n++) {\n` +
    `    let _acc_1 = out[m * ${N} + n];\n` +
    `    for (let k = 0; k < ${K}; k++) {\n` +
    `      _acc_1 = (_acc_1 + (${a} * ${b}));\n    }\n` +
    `    out[m * ${N} + n] = _acc_1;\n  }\n}`;
  return new Function('A', 'B', 'out', src);
}

// convert -> broadcast_in_dim(sv) -> mul [-> add bias] [-> max 0], fused.
function buildEpiloguePerChannel(M, N, withBias, relu) {
  let v = `Math.fround((+acc[m * ${N} + n]) * sv[n])`;
  if (withBias) v = `Math.fround(${v} + bias[n])`;
  if (relu) v = `Math.max(${v}, 0)`;
  const src = `for (let m = 0; m < ${M}; m++) {\n  for (let n = 0; n < ${N}; n++) {\n` +
    `    y[m * ${N} + n] = ${v};\n  }\n}`;
  return new Function('acc', 'sv', 'bias', 'y', src);
}

// silu(x) = x * (1 / (1 + exp(-x))) decomposed (decomposition_pass.ts:197-230)
function buildSiluMul(n) {
  const src = `for (let i = 0; i < ${n}; i++) {\n` +
    `  const x = g[i];\n` +
    `  h[i] = Math.fround(Math.fround(x * Math.fround(1 / Math.fround(1 + Math.fround(Math.exp((-x)))))) * u[i]);\n}`;
  return new Function('g', 'u', 'h', src);
}

// ---- CLI ---------------------------------------------------------------
// node q8ref.js <cmd> '<json params>' [in files...] -- [out files...]
const DT = { f32: Float32Array, f64: Float64Array, i8: Int8Array, u8: Uint8Array, i32: Int32Array };

function readArr(path, dt) {
  const buf = fs.readFileSync(path);
  const ab = buf.buffer.slice(buf.byteOffset, buf.byteOffset + buf.byteLength);
  return new DT[dt](ab);
}
function writeArr(path, arr) {
  fs.writeFileSync(path, Buffer.from(arr.buffer, arr.byteOffset, arr.byteLength));
}

function hr() { return Number(process.hrtime.bigint()) / 1e9; }

function timeIt(fn, reps) {
  fn();                                  // one JIT warm-up run
  const t = [];
  for (let r = 0; r < reps; r++) { const t0 = hr(); fn(); t.push(hr() - t0); }
  t.sort((a, b) => a - b);
  return t[Math.floor(t.length / 2)];
}

function main(argv) {
  const cmd = argv[0];
  const p = argv[1] ? JSON.parse(argv[1]) : {};
  const files = argv.slice(2);
  const sep = files.indexOf('--');
  const ins = sep >= 0 ? files.slice(0, sep) : files;
  const outs = sep >= 0 ? files.slice(sep + 1) : [];

  if (cmd === 'rng') {                 // raw draws
    const rng = makeRng(p.seed);
    const o = new Float64Array(p.n);
    for (let i = 0; i < p.n; i++) o[i] = rng();
    writeArr(outs[0], o);
  } else if (cmd === 'normal' || cmd === 'uniform') {
    const rng = makeRng(p.seed);
    const o = new Float32Array(p.n);
    if (cmd === 'normal') normalFill(rng, o, p.mean, p.std); else uniformFill(rng, o, p.a, p.b);
    writeArr(outs[0], o);
  } else if (cmd === 'quantize') {
    const x = readArr(ins[0], 'f32');
    const q = p.unsigned ? new Uint8Array(x.length) : new Int8Array(x.length);
    buildQuantize(x.length, p.scale, p.zero_point || 0, !!p.unsigned)(x, q);
    writeArr(outs[0], q);
  } else if (cmd === 'quantize_rows') {
    const x = readArr(ins[0], 'f32'), sc = readArr(ins[1], 'f64');
    const q = new Int8Array(p.M * p.K);
    buildQuantizeRows(p.M, p.K)(x, sc, q);
    writeArr(outs[0], q);
  } else if (cmd === 'scales_rows') {
    const x = readArr(ins[0], 'f32');
    writeArr(outs[0], scalesPerToken(x, p.M, p.K, new Float64Array(p.M)));
  } else if (cmd === 'dequantize') {
    const q = readArr(ins[0], p.src || 'i8');
    const y = new Float32Array(q.length);
    buildDequantize(q.length, p.scale, p.zero_point || 0)(q, y);
    writeArr(outs[0], y);
  } else if (cmd === 'dequantize_rows') {
    const q = readArr(ins[0], 'i8'), sc = readArr(ins[1], 'f64');
    const y = new Float32Array(p.M * p.K);
    buildDequantizeRows(p.M, p.K)(q, sc, y);
    writeArr(outs[0], y);
  } else if (cmd === 'qdot') {
    const A = readArr(ins[0], 'i8'), B = readArr(ins[1], 'i8');
    const out = new Int32Array(p.M * p.N);
    buildQuantizedDot(p.M, p.N, p.K, p.b_layout, p.zpA || 0, p.zpB || 0)(A, B, out);
    writeArr(outs[0], out);
  } else if (cmd === 'epilogue_pc') {
    const acc = readArr(ins[0], 'i32'), sv = readArr(ins[1], 'f32');
    const bias = ins[2] ? readArr(ins[2], 'f32') : null;
    const y = new Float32Array(p.M * p.N);
    buildEpiloguePerChannel(p.M, p.N, !!bias, !!p.relu)(acc, sv, bias, y);
    writeArr(outs[0], y);
  } else if (cmd === 'silu_mul') {
    const g = readArr(ins[0], 'f32'), u = readArr(ins[1], 'f32');
    const h = new Float32Array(g.length);
    buildSiluMul(g.length)(g, u, h);
    writeArr(outs[0], h);
  } else if (cmd === 'bench') {
    // Timed CPU baseline on synthetic data of the requested shape.
    // kind: 'qdot' (M rows of an M x N x K qmatmul + per-channel epilogue),
    //       'quantize_rows', 'dequantize_rows'.
    const rng = makeRng(p.seed >>> 0);
    const reps = p.reps || 5;
    const res = { kind: p.kind, cores: 1, node: process.version };
    if (p.kind === 'qdot') {
      const A = new Int8Array(p.M * p.K), B = new Int8Array(p.N * p.K);
      for (let i = 0; i < A.length; i++) A[i] = (rng() * 255 - 127) | 0;
      for (let i = 0; i < B.length; i++) B[i] = (rng() * 255 - 127) | 0;
      const acc = new Int32Array(p.M * p.N);
      const sv = new Float32Array(p.N).fill(1e-4);
      const y = new Float32Array(p.M * p.N);
      const dot = buildQuantizedDot(p.M, p.N, p.K, 1, 0, 0);
      const epi = buildEpiloguePerChannel(p.M, p.N, false, false);
      res.seconds = timeIt(() => { dot(A, B, acc); epi(acc, sv, null, y); }, reps);
      res.ops = 2 * p.M * p.N * p.K;
    } else if (p.kind === 'quantize_rows' || p.kind === 'dequantize_rows') {
      const x = normalFill(rng, new Float32Array(p.M * p.K), 0, 1);
      const sc = new Float64Array(p.M);
      for (let m = 0; m < p.M; m++) {
        let mn = Infinity, mx = -Infinity;
        for (let k = 0; k < p.K; k++) { const v = x[m * p.K + k]; if (v < mn) mn = v; if (v > mx) mx = v; }
        sc[m] = Math.max(Math.abs(mn), Math.abs(mx)) / 127 || 1e-10;
      }
      const q = new Int8Array(p.M * p.K);
      const qz = buildQuantizeRows(p.M, p.K);
      if (p.kind === 'quantize_rows') {
        res.seconds = timeIt(() => qz(x, sc, q), reps);
      } else {
        qz(x, sc, q);
        const y = new Float32Array(p.M * p.K);
        const dq = buildDequantizeRows(p.M, p.K);
        res.seconds = timeIt(() => dq(q, sc, y), reps);
      }
      res.bytes = p.M * p.K * 5 + p.M * 8;
    } else {
      throw new Error('unknown bench kind ' + p.kind);
    }
    process.stdout.write(JSON.stringify(res) + '\n');
  } else {
    throw new Error('unknown command ' + cmd);
  }
}

if (require.main === module) main(process.argv.slice(2));

module.exports = {
  makeRng, normalFill, uniformFill, buildQuantize, buildQuantizeRows, scalesPerToken, buildDequantize,
  buildDequantizeRows, buildQuantizedDot, buildEpiloguePerChannel, buildSiluMul,
};
