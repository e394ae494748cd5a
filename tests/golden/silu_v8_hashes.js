// SiLU as the reference's CPU backend evaluates it (decomposition_pass.ts:
// 197-230 lowered to JS: every f32 op rounded with Math.fround, exp in f64),
// over every binary32 input, hashed per chunk of 2^24 consecutive bit
// patterns.  Per chunk c (inputs with bits c * 2^24 + i):
//   v_i = bit pattern of silu(x_i), any NaN as 0x7fc00000
//   m_i = mix(v_i): v ^= v >>> 16; v *= 0x7feb352d; v ^= v >>> 15 (mod 2^32,
//         a bijection, so a change of any size in any element shows)
//   s1  = sum_i m_i * (2i + 1)  mod 2^32
//   s2  = sum_i m_i             mod 2^32
// Usage: node silu_v8_hashes.js <first chunk> <end chunk>  ->  JSON lines
'use strict';
const first = parseInt(process.argv[2], 10), end = parseInt(process.argv[3], 10);
const u32 = new Uint32Array(1), f32 = new Float32Array(u32.buffer);
function silu(x) {
  return Math.fround(x * Math.fround(1 / Math.fround(1 + Math.fround(Math.exp(-x)))));
}
for (let c = first; c < end; c++) {
  let s1 = 0, s2 = 0;
  const base = c * 16777216;
  for (let i = 0; i < 16777216; i++) {
    u32[0] = base + i;
    f32[0] = silu(f32[0]);
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
