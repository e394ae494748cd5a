// The compiled quantize R1 (quant_math.ts:16-27 as the CPU backend emits it:
// (Math.min(Math.max(Math.round(Math.fround(x / S)), -128), 127) | 0)) over
// every binary32 input x, for one scale S, hashed per chunk of 2^24
// consecutive bit patterns.  Per chunk c (inputs with bits c * 2^24 + i):
//   v_i = the code's byte (code & 0xff)
//   m_i = mix(v_i): v ^= v >>> 16; v *= 0x7feb352d; v ^= v >>> 15 (mod 2^32)
//   s1  = sum_i m_i * (2i + 1)  mod 2^32
//   s2  = sum_i m_i             mod 2^32
// Usage: node quant_v8_hashes.js <scale> <first chunk> <end chunk>  ->  JSON lines
'use strict';
const S = parseFloat(process.argv[2]);
const first = parseInt(process.argv[3], 10), end = parseInt(process.argv[4], 10);
const u32 = new Uint32Array(1), f32 = new Float32Array(u32.buffer);
const MIX = new Uint32Array(256);
for (let b = 0; b < 256; b++) {
  let v = b;
  v = (v ^ (v >>> 16)) >>> 0;
  v = Math.imul(v, 0x7feb352d) >>> 0;
  MIX[b] = (v ^ (v >>> 15)) >>> 0;
}
for (let c = first; c < end; c++) {
  let s1 = 0, s2 = 0;
  const base = c * 16777216;
  for (let i = 0; i < 16777216; i++) {
    u32[0] = base + i;
    const x = f32[0];
    const q = (Math.min(Math.max(Math.round(Math.fround(x / S)), -128), 127) | 0);
    const m = MIX[q & 0xff];
    s1 = (s1 + Math.imul(m, 2 * i + 1)) | 0;
    s2 = (s2 + m) | 0;
  }
  process.stdout.write(JSON.stringify([c, s1 >>> 0, s2 >>> 0]) + '\n');
}
