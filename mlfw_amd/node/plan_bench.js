'use strict';
/*
 * Per-call cost of whole quantized plans through the Node drop-in: the
 * 'hip' runtime backend's runPlan (hip_backend.js) over the N-API addon,
 * timed on the host around each call (host work, uploads, launches, the
 * final synchronization and downloads included), as the reference's
 * runPlanAsync drives its CUDA plan runner (runtime.ts:290-329,
 * device_plan.ts:178-297).
 *
 * Plans are the PrimFunc sets QuantizationPass and the lowering rules leave
 * for a chain of per-channel linears (quantize -> [quantized_dot ->
 * convert*mul(sv) + bias (-> max 0 -> quantize)]*), built with
 * tir_build.js and compiled by the hip external codegen:
 *   c2:     the C2 MLP, batch 256, 784 -> 256 -> 128 -> 10, ReLU and a static
 *           requant between layers, f32 logits;
 *   decode: four 4096 x 4096 linears for one token (M = 1).
 * Each plan runs eagerly and as a replayed HIP graph, with its inputs
 * uploaded every call and with them resident (RuntimeTensor.resident pins,
 * runPlan {resident: true}).
 *
 *   node plan_bench.js [calls]      prints one JSON object
 */
const path = require('path');
const hip = require('./hip_backend.js');
const A = require('./index.js');
const T = require('./tir_build.js');

function lcg(seed) {
  let s = seed >>> 0;
  return () => { s = (Math.imul(s, 1664525) + 1013904223) >>> 0; return s / 4294967296; };
}
function randI8(seed, n) { const r = lcg(seed), a = new Int8Array(n); for (let i = 0; i < n; i++) a[i] = Math.floor(r() * 255) - 127; return a; }
function randF32(seed, n, lo, hi) { const r = lcg(seed), a = new Float32Array(n); for (let i = 0; i < n; i++) a[i] = lo + r() * (hi - lo); return a; }

/** A chain of per-channel linears dims[0] -> dims[1] -> ... for M tokens. */
function chainPlan(M, dims, seed) {
  const provider = hip.createHipProvider('external_codegen', 'const_buffers');
  const codegen = hip.createHipExternalCodegen('const_buffers');
  const kernelOf = (pf) => { provider.annotate([pf]); return codegen.compile(pf, hip.hipTarget(), pf.getAttr('external_codegen').info); };
  const { buf, math, ext, cast, pointwise, quantizeExpr, qmatmulPF } = T;
  const L = dims.length - 1;
  const sIn = [4.0 / 127];
  for (let i = 1; i < L; i++) sIn.push(0.05 * i);
  const x = buf('x', [M, dims[0]], 'f32'), q0 = buf('q0', [M, dims[0]], 'i8');
  const steps = [], slots = [];
  const slot = (data, shape, dtype) => { slots.push({ data, shape, dtype }); return slots.length - 1; };
  const S = (pf, ins, outs) => steps.push({ name: pf.name, inputSlots: ins, outputSlots: outs, kernel: kernelOf(pf), shapeValues: null });
  const xSlot = slot(randF32(seed, M * dims[0], -3, 3), [M, dims[0]], 'f32');
  const bSlots = [];
  for (let i = 0; i < L; i++) bSlots.push(slot(randF32(seed + 100 + i, dims[i + 1], -0.1, 0.1), [dims[i + 1]], 'f32'));
  let qSlot = slot(new Int8Array(M * dims[0]), [M, dims[0]], 'i8');
  S(pointwise('quantize', q0, [x], (l) => quantizeExpr(l[0], sIn[0])), [xSlot], [qSlot]);
  let qBuf = q0, outSlot = -1;
  for (let i = 0; i < L; i++) {
    const K = dims[i], N = dims[i + 1], last = i === L - 1;
    const W = buf(`w${i}`, [N, K], 'i8'), acc = buf(`acc${i}`, [M, N], 'i32');
    const sv = buf(`sv${i}`, [N], 'f32'), b = buf(`b${i}`, [N], 'f32'), zero = buf(`zero${i}`, [1, 1], 'f32');
    const out = buf(`o${i}`, [M, N], last ? 'f32' : 'i8');
    const svd = new Float32Array(N);
    for (let n = 0; n < N; n++) svd[n] = Math.fround(sIn[i] * (0.5 + (n % 7) / 7) / (127 * Math.sqrt(K)));
    const cW = { buffer: W, data: randI8(seed + 10 + i, N * K) }, cS = { buffer: sv, data: svd };
    const cZ = { buffer: zero, data: new Float32Array([0]) };
    const lin = (l) => math('+', math('*', cast(l[0], 'i32', 'f32'), l[1]), l[2]);
    const epi = last ? pointwise(`tail${i}`, out, [acc, sv, b], lin, [cS])
                     : pointwise(`relu_rq${i}`, out, [acc, sv, b, zero], (l) => quantizeExpr(ext('max', [lin(l), l[3]]), sIn[i + 1]), [cS, cZ]);
    const accSlot = slot(new Int32Array(M * N), [M, N], 'i32');
    const oSlot = slot(last ? new Float32Array(M * N) : new Int8Array(M * N), [M, N], last ? 'f32' : 'i8');
    S(qmatmulPF(M, N, K, qBuf, W, acc, [cW]), [qSlot], [accSlot]);
    S(epi, [accSlot, bSlots[i]], [oSlot]);
    qBuf = out;
    qSlot = oSlot;
    outSlot = oSlot;
  }
  const plan = { numSlots: slots.length, argSlots: [xSlot, ...bSlots, outSlot], intermediates: [],
                 steps: steps.map((s) => ({ name: s.name, inputSlots: s.inputSlots, outputSlots: s.outputSlots })) };
  return { plan, slots, steps, xSlot, bSlots, outSlot };
}

function timeCalls(c, opts, calls, warm) {
  for (let i = 0; i < warm; i++) hip.runPlanSync(c.plan, c.slots, c.steps, opts);
  hip.resetStats();
  const t0 = process.hrtime.bigint();
  for (let i = 0; i < calls; i++) hip.runPlanSync(c.plan, c.slots, c.steps, opts);
  const t1 = process.hrtime.bigint();
  const per = (v) => v / calls;
  return {
    us_per_call: Number(t1 - t0) / 1e3 / calls,
    upload_bytes_per_call: per(hip.stats.uploadBytes),
    download_bytes_per_call: per(hip.stats.downloadBytes),
    launches_per_call: per(hip.stats.launches),
    graph_replays_per_call: per(hip.stats.graphReplays),
  };
}

function benchPlan(c, calls) {
  const res = {};
  // every input re-sent each call (x and the biases are plain arguments)
  res.eager = timeCalls(c, { graph: false }, calls, 5);
  const want = c.slots[c.outSlot].data.slice();
  res.graph = timeCalls(c, { graph: true }, calls, 5);
  const got = c.slots[c.outSlot].data;
  res.graph_output_equals_eager = Buffer.compare(Buffer.from(got.buffer, got.byteOffset, got.byteLength),
                                                 Buffer.from(want.buffer, want.byteOffset, want.byteLength)) === 0;
  // inputs pinned resident: a call with unchanged arguments uploads nothing
  for (const s of [c.xSlot, ...c.bSlots]) c.slots[s].resident = { key: c.slots[s].data, version: 1 };
  res.graph_resident = timeCalls(c, { graph: true, resident: true }, calls, 2);
  res.eager_resident = timeCalls(c, { graph: false, resident: true }, calls, 2);
  hip.releasePlan(c.plan);
  return res;
}

function main() {
  const calls = Number(process.argv[2] || 200);
  A.init(0);
  const out = { calls, node: process.version };
  out.c2_mlp_b256 = benchPlan(chainPlan(256, [784, 256, 128, 10], 1), calls);
  out.decode_m1_4x4096 = benchPlan(chainPlan(1, [4096, 4096, 4096, 4096, 4096], 2), calls);
  console.log(JSON.stringify(out));
}

main();
