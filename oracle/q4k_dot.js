'use strict';
// CPU baseline (test infrastructure, run by bench.py's cpu_baseline leg only):
// the config-0 Q4_K GEMV y[M] = W[M, K] . x[K] as a TypeScript host would run
// it in Node, on one core, in plain ES2019 (no TypeScript compiler here).
// It restates GGUFParser.dequantizeQ4_K (src/gguf.ts:168-210: per 144-byte
// block d, dmin, 12 bytes of 6-bit scale/min pairs, 128 bytes of nibbles;
// element = d*sc*q - dmin*m stored as f32) and the matvec of
// shaders/matmul_quant.wgsl:21-54 (one dot product per row).
//
// usage: node q4k_dot.js <input.bin> <output.bin> <seconds>
//   input.bin:  u32 M, u32 K, then M*K/256 Q4_K blocks, then K f32 x
//   output.bin: M f32 y (from the dequant-in-the-loop variant)
// Prints one JSON line: per-GEMV milliseconds with the dequant inside the
// timed loop (the whole weight matrix decoded from the raw blocks on every
// GEMV) and with the matrix decoded once beforehand (f32 dot only).

const fs = require('fs');

function f16ToF32(h) {
  const s = (h & 0x8000) ? -1 : 1;
  const e = (h >> 10) & 0x1f;
  const m = h & 0x3ff;
  if (e === 0) return s * m * Math.pow(2, -24);
  if (e === 31) return m ? NaN : s * Infinity;
  return s * (1 + m / 1024) * Math.pow(2, e - 15);
}

// One row of nb blocks starting at byte `off` of `buf` into out[0 .. 256 nb).
function dequantRow(buf, off, nb, out) {
  let o = 0;
  for (let b = 0; b < nb; b++, off += 144) {
    const d = f16ToF32(buf[off] | (buf[off + 1] << 8));
    const dmin = f16ToF32(buf[off + 2] | (buf[off + 3] << 8));
    const s = off + 4;
    const q = off + 16;
    for (let g = 0; g < 4; g++) {
      const j0 = 2 * g, j1 = 2 * g + 1;
      let sc0, m0, sc1, m1;
      if (j0 < 4) {
        sc0 = buf[s + j0] & 63; m0 = buf[s + j0 + 4] & 63;
      } else {
        sc0 = (buf[s + j0 + 4] & 15) | ((buf[s + j0 - 4] >> 6) << 4);
        m0 = (buf[s + j0 + 4] >> 4) | ((buf[s + j0] >> 6) << 4);
      }
      if (j1 < 4) {
        sc1 = buf[s + j1] & 63; m1 = buf[s + j1 + 4] & 63;
      } else {
        sc1 = (buf[s + j1 + 4] & 15) | ((buf[s + j1 - 4] >> 6) << 4);
        m1 = (buf[s + j1 + 4] >> 4) | ((buf[s + j1] >> 6) << 4);
      }
      const d0 = d * sc0, n0 = dmin * m0, d1 = d * sc1, n1 = dmin * m1;
      const qg = q + 32 * g;
      for (let l = 0; l < 32; l++) out[o + l] = d0 * (buf[qg + l] & 15) - n0;
      for (let l = 0; l < 32; l++) out[o + 32 + l] = d1 * (buf[qg + l] >> 4) - n1;
      o += 64;
    }
  }
}

function dot(w, wo, x, K) {
  let acc = 0;
  for (let k = 0; k < K; k++) acc += w[wo + k] * x[k];
  return acc;
}

function main() {
  const [inPath, outPath, secs] = process.argv.slice(2);
  const raw = fs.readFileSync(inPath);
  const buf = new Uint8Array(raw.buffer, raw.byteOffset, raw.length);
  const hdr = new Uint32Array(raw.buffer.slice(raw.byteOffset, raw.byteOffset + 8));
  const M = hdr[0], K = hdr[1], nb = K / 256, rowBytes = nb * 144;
  const wOff = 8;
  const xb = raw.buffer.slice(raw.byteOffset + wOff + M * rowBytes, raw.byteOffset + wOff + M * rowBytes + 4 * K);
  const x = new Float32Array(xb);
  const y = new Float32Array(M);
  const row = new Float32Array(K);
  const budgetNs = BigInt(Math.round(Number(secs) * 1e9));

  // dequant inside the loop
  let reps = 0;
  const t0 = process.hrtime.bigint();
  let t1 = t0;
  do {
    for (let m = 0; m < M; m++) {
      dequantRow(buf, wOff + m * rowBytes, nb, row);
      y[m] = dot(row, 0, x, K);
    }
    reps++;
    t1 = process.hrtime.bigint();
  } while (t1 - t0 < budgetNs);
  const msDequant = Number(t1 - t0) / 1e6 / reps;
  fs.writeFileSync(outPath, Buffer.from(y.buffer));

  // pre-dequantized f32 matrix, dot only
  const W = new Float32Array(M * K);
  for (let m = 0; m < M; m++) {
    dequantRow(buf, wOff + m * rowBytes, nb, row);
    W.set(row, m * K);
  }
  let reps2 = 0;
  const t2 = process.hrtime.bigint();
  let t3 = t2;
  let chk = 0;
  do {
    for (let m = 0; m < M; m++) y[m] = dot(W, m * K, x, K);
    chk += y[0];
    reps2++;
    t3 = process.hrtime.bigint();
  } while (t3 - t2 < budgetNs);
  const msDot = Number(t3 - t2) / 1e6 / reps2;
  console.log(JSON.stringify({ M: M, K: K, reps_dequant: reps, ms_dequant_dot: msDequant,
                               reps_dot: reps2, ms_dot_predequantized: msDot, node: process.version,
                               check: chk }));
}

main();
