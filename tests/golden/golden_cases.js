'use strict';
/*
 * Golden vectors for the int8 path, computed in a JavaScript engine (V8)
 * with the reference's arithmetic, so the expectations come from the
 * engine's own Math.round / Math.fround / typed-array semantics rather than
 * from the C oracle they are used to check.
 *
 * Cases (reference file:line they restate):
 *   params     tests/compiler/passes/quantization/params.test.js:5-233 inputs
 *              through fromRange / fromConstantArray / per-channel / per-group
 *              scale rules (src/compiler/ir/graph/quantization_types.ts:248-340)
 *              and the host quantize (:75-79, :118-130)
 *   fakequant  pass.test.js:461-491: compiled quantize -> dequantize of
 *              [3.5, -2.1, 5.9, 1.234, -5.9, 0.001] at scale 6/127
 *   pcmatmul   pass.test.js:493-549: per-channel and per-tensor int8 matmul of
 *              sin-valued A [4,8] and skewed W [8,6] (rhs_contracting = [0])
 *   edges      compiled quantize of special values at several scales
 *   c1         BASELINE config C1 (seed 0) end to end
 * Usage: node golden_cases.js <out_dir>   (writes <case>.json / <name>.bin)
 */
const fs = require('fs');
const path = require('path');
const K = require(path.join(__dirname, '..', '..', 'oracle', 'q8ref.js'));

const out = process.argv[2];
const writeBin = (name, arr) => fs.writeFileSync(path.join(out, name + '.bin'),
                                                Buffer.from(arr.buffer, arr.byteOffset, arr.byteLength));

// scale rules, quantization_types.ts:248-317
function symScale(mn, mx, bits) {
  return Math.max(Math.abs(mn), Math.abs(mx)) / (2 ** (bits - 1) - 1) || 1e-10;
}
function asymParams(mn, mx, unsigned, bits) {
  const cMin = unsigned ? 0 : -(2 ** (bits - 1)), cMax = unsigned ? 2 ** bits - 1 : 2 ** (bits - 1) - 1;
  const s = (mx - mn || 1e-10) / (cMax - cMin);
  return { scale: s, zeroPoint: Math.max(cMin, Math.min(cMax, Math.round(cMin - mn / s))) };
}
function rangeOf(arr) {
  let mn = Infinity, mx = -Infinity;
  for (const v of arr) { if (v < mn) mn = v; if (v > mx) mx = v; }
  if (!isFinite(mn)) mn = -1;
  if (!isFinite(mx)) mx = 1;
  if (mn === mx) { mn -= 0.5; mx += 0.5; }
  return [mn, mx];
}
function hostQuant(v, s, zp, lo, hi) { return Math.max(lo, Math.min(hi, Math.round(v / s + zp))); }
function perChannelScales(W, rows, cols, axis, bits) {
  const nch = axis === 0 ? rows : cols, s = new Float64Array(nch);
  for (let c = 0; c < nch; c++) {
    const vals = [];
    for (let j = 0; j < (axis === 0 ? cols : rows); j++) vals.push(axis === 0 ? W[c * cols + j] : W[j * cols + c]);
    const [mn, mx] = rangeOf(vals);
    s[c] = symScale(mn, mx, bits);
  }
  return s;
}

fs.mkdirSync(out, { recursive: true });

// ---------------------------------------------------------------- params
{
  const r = {};
  r.sym = [[-3, 3], [-1, 5], [-6, 6], [-1, 1], [-10, 10], [-5, 5]].map(([a, b]) => symScale(a, b, 8));
  r.asym_i8_0_6 = asymParams(0, 6, false, 8);
  r.asym_u8_0_1 = asymParams(0, 1, true, 8);
  r.const_1m2_3 = symScale(...rangeOf(Float32Array.from([1, -2, 3, -0.5])), 8);
  r.const_555 = symScale(...rangeOf(Float32Array.from([5, 5, 5])), 8);
  const s66 = symScale(-6, 6, 8), s11 = symScale(-1, 1, 8), s1010 = symScale(-10, 10, 8);
  r.q_3p5 = hostQuant(3.5, s66, 0, -127, 127);
  r.q_pm1000 = [hostQuant(1000, s11, 0, -127, 127), hostQuant(-1000, s11, 0, -127, 127)];
  r.q_array = Array.from(Float32Array.from([1.5, -3.2, 0.0, 7.8]), (v) => hostQuant(v, s1010, 0, -127, 127));
  const Ks = 4, Ns = 3, W = new Float32Array(Ks * Ns);
  for (let k = 0; k < Ks; k++) for (let n = 0; n < Ns; n++) W[k * Ns + n] = Math.sin(k * 1.7 + n) * (n + 1) * 3;
  writeBin('params_skewed_W', W);
  const sc1 = perChannelScales(W, Ks, Ns, 1, 8), sc0 = perChannelScales(W, Ks, Ns, 0, 8);
  r.pc_axis1 = Array.from(sc1);
  r.pc_axis0 = Array.from(sc0);
  r.pc_axis1_q = Array.from(W, (v, i) => hostQuant(v, sc1[i % Ns], 0, -128, 127));
  const G = 16, data = new Float32Array(64);
  for (let i = 0; i < 64; i++) data[i] = Math.sin(i * 0.9) * (1 + (i % G) * 0.1);
  writeBin('params_group_data', data);
  const gs = [];
  for (let g = 0; g < 4; g++) {
    let a = 0;
    for (let i = g * G; i < (g + 1) * G; i++) a = Math.max(a, Math.abs(data[i]));
    gs.push(a / 7 || 1e-10);
  }
  r.group_scales = gs;
  r.group_q = Array.from(data, (v, i) => hostQuant(v, gs[Math.floor(i / G)], 0, -7, 7));
  fs.writeFileSync(path.join(out, 'params.json'), JSON.stringify(r));
}

// ---------------------------------------------------------------- fake quant
{
  const s = symScale(-6, 6, 8);
  const x = Float32Array.from([3.5, -2.1, 5.9, 1.234, -5.9, 0.001]);
  const q = new Int8Array(x.length), y = new Float32Array(x.length);
  K.buildQuantize(x.length, s, 0, false)(x, q);
  K.buildDequantize(x.length, s, 0)(q, y);
  writeBin('fakequant_x', x); writeBin('fakequant_q', q); writeBin('fakequant_y', y);
  fs.writeFileSync(path.join(out, 'fakequant.json'), JSON.stringify({ scale: s }));
}

// ---------------------------------------------------------------- per-channel matmul
{
  const M = 4, Kd = 8, N = 6;
  const A = new Float32Array(M * Kd);
  for (let i = 0; i < A.length; i++) A[i] = Math.sin(i * 0.7);
  const W = new Float32Array(Kd * N);
  for (let k = 0; k < Kd; k++) for (let n = 0; n < N; n++) W[k * N + n] = Math.sin(k * 1.3 + n) * (n + 1) * 2;
  let aMax = 0;
  for (const v of A) aMax = Math.max(aMax, Math.abs(v));
  const aScale = aMax / 127 || 1e-10;
  const aq = new Int8Array(M * Kd);
  K.buildQuantize(A.length, aScale, 0, false)(A, aq);
  const results = {};
  for (const mode of ['pc', 'pt']) {
    let wq, sv;
    if (mode === 'pc') {
      const sc = perChannelScales(W, Kd, N, 1, 8);
      wq = Int8Array.from(W, (v, i) => hostQuant(v, sc[i % N], 0, -128, 127));
      sv = Float32Array.from(sc, (s) => aScale * s);
    } else {
      const s = symScale(...rangeOf(W), 8);
      wq = Int8Array.from(W, (v) => hostQuant(v, s, 0, -127, 127));
      sv = new Float32Array(N).fill(aScale * s);
    }
    const acc = new Int32Array(M * N), y = new Float32Array(M * N);
    K.buildQuantizedDot(M, N, Kd, 0, 0, 0)(aq, wq, acc);
    K.buildEpiloguePerChannel(M, N, false, false)(acc, sv, null, y);
    writeBin(`pcmatmul_${mode}_wq`, wq); writeBin(`pcmatmul_${mode}_acc`, acc); writeBin(`pcmatmul_${mode}_y`, y);
    results[mode] = { sv: Array.from(sv) };
  }
  writeBin('pcmatmul_A', A); writeBin('pcmatmul_W', W); writeBin('pcmatmul_aq', aq);
  fs.writeFileSync(path.join(out, 'pcmatmul.json'), JSON.stringify({ aScale, ...results }));
}

// ---------------------------------------------------------------- edge values
{
  const x = Float32Array.from([NaN, Infinity, -Infinity, -0, 0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 127.49,
                               127.5, -128.5, -128.51, 1e30, -1e30, 1e-40, -1e-40, 0.11811023205518723,
                               -0.11811023205518723, 3.4e38, 0.001]);
  const scales = [1, 6 / 127, 0.0123, 1e-10, 3];
  writeBin('edges_x', x);
  scales.forEach((s, j) => {
    const q = new Int8Array(x.length), u = new Uint8Array(x.length);
    K.buildQuantize(x.length, s, 0, false)(x, q);
    K.buildQuantize(x.length, s, 0, true)(x, u);
    writeBin(`edges_q_${j}`, q); writeBin(`edges_u_${j}`, u);
  });
  fs.writeFileSync(path.join(out, 'edges.json'), JSON.stringify({ scales }));
}

// ---------------------------------------------------------------- C1
{
  const rng = K.makeRng(0);
  const M = 32, Kd = 128, N = 64;
  const X = K.normalFill(rng, new Float32Array(M * Kd), 0, 1);
  const W = K.normalFill(rng, new Float32Array(N * Kd), 0, 0.02);
  const bias = K.uniformFill(rng, new Float32Array(N), -0.1, 0.1);
  let mn = Infinity, mx = -Infinity;
  for (const v of X) { if (v < mn) mn = v; if (v > mx) mx = v; }
  const sX = symScale(mn, mx, 8);
  const sW = perChannelScales(W, N, Kd, 0, 8);
  const Wq = Int8Array.from(W, (v, i) => hostQuant(v, sW[Math.floor(i / Kd)], 0, -128, 127));
  const Xq = new Int8Array(M * Kd);
  K.buildQuantize(X.length, sX, 0, false)(X, Xq);
  const acc = new Int32Array(M * N), y = new Float32Array(M * N);
  K.buildQuantizedDot(M, N, Kd, 1, 0, 0)(Xq, Wq, acc);
  const sv = Float32Array.from(sW, (s) => sX * s);
  K.buildEpiloguePerChannel(M, N, true, false)(acc, sv, bias, y);
  for (const [n, a] of [['c1_X', X], ['c1_W', W], ['c1_bias', bias], ['c1_Xq', Xq], ['c1_Wq', Wq],
                        ['c1_sW', sW], ['c1_acc', acc], ['c1_y', y]]) writeBin(n, a);
  fs.writeFileSync(path.join(out, 'c1.json'), JSON.stringify({ sX }));
}
console.log('golden cases written to ' + out);
