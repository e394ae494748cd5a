// Math.fround(Math.<fn>(x)) -- the reference CPU backend's emission of an
// f32-typed exp / log / tanh extern (src/backend/cpu/codegen.ts:534: a
// non-exact extern is wrapped in Math.fround; the expected string
// 'Math.fround(Math.exp(x))' of tests/backend/cpu/codegen-internals.test.js)
// -- over every binary32 input, hashed per chunk of 2^24 consecutive bit
// patterns with the definitions of silu_v8_hashes.js:
//   v_i = bit pattern of the result, any NaN as 0x7fc00000
//   m_i = mix(v_i): v ^= v >>> 16; v *= 0x7feb352d; v ^= v >>> 15 (mod 2^32)
//   s1  = sum_i m_i * (2i + 1)  mod 2^32,  s2 = sum_i m_i  mod 2^32
// Usage: node ewise_v8_hashes.js <exp|log|tanh> <first chunk> <end chunk>  ->  JSON lines
'use strict';
const name = process.argv[2];
const first = parseInt(process.argv[3], 10), end = parseInt(process.argv[4], 10);
const fns = { exp: (x) => Math.fround(Math.exp(x)), log: (x) => Math.fround(Math.log(x)),
              tanh: (x) => Math.fround(Math.tanh(x)) };
const fn = fns[name];
if (!fn) { console.error(`unknown function ${name}`); process.exit(2); }
const u32 = new Uint32Array(1), f32 = new Float32Array(u32.buffer);
for (let c = first; c < end; c++) {
  let s1 = 0, s2 = 0;
  const base = c * 16777216;
  for (let i = 0; i < 16777216; i++) {
    u32[0] = base + i;
    f32[0] = fn(f32[0]);
    let v = u32[0];
    if ((v & 0x7f800000) === 0x7f800000 && (v & 0x007fffff) !== 0) v = 0x7fc00000;
    v = (v ^ (v >>> 16)) >>> 0;
    v = Math.imul(v, 0x7feb352d) >>> 0;
    v = (v ^ (v >>> 15)) >>> 0;
    s1 = (s1 + Math.imul(v, 2 * i + 1)) | 0;
    s2 = (s2 + v) | 0;
  }
  process.stdout.write(JSON.stringify([c, s1 >>> 0, s2 >>> 0]) + '\n');
}
