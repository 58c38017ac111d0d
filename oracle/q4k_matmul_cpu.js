'use strict';
// TEST INFRASTRUCTURE ONLY: the CPU baseline that bench.py times beside the
// GPU (and the tests check against the C oracle). Never part of the product.
//
// Plain-JavaScript restatement of the reference's CPU check of the Q4_K
// dequant-matmul: every weight row decoded the way dequantizeQ4KBlock does
// (src/gguf/quantization.ts:2-38: binary16 d and dmin, 6-bit scale/min pairs
// of scaleAndMin, out = d * sc * q - dmin * m evaluated in double and stored
// to a Float32Array), then a scalar double-precision dot with each input row
// (src/main.ts:97-104), here for every element of Y = X W^T instead of the
// one element the reference checks.
//
// node q4k_matmul_cpu.js <W.bin> <X_f16.bin> <m> <n> <k> <runs> [<Y_out.bin>]
//   W: n rows of k/256 Q4_K blocks (144 bytes); X: m x k binary16 values.
// Prints one JSON line: per-run milliseconds, their median, Node version and
// a float64 checksum; with an output path, also writes Y as float64.
const fs = require('fs');

// IEEE 754 binary16 bits -> number (subnormals, infinities, NaN).
function halfBitsToNumber(bits) {
  const negative = (bits & 0x8000) !== 0;
  const e = (bits >> 10) & 31;
  const f = bits & 1023;
  let v;
  if (e === 0) v = f * Math.pow(2, -24);
  else if (e === 31) v = f ? NaN : Infinity;
  else v = (1024 + f) * Math.pow(2, e - 25);
  return negative ? -v : v;
}

// Sub-block j of a block's 12 packed scale bytes at s[o..o+11] -> [scale, min]:
// j < 4 keeps the low 6 bits of bytes j and j + 4; j >= 4 joins the nibbles
// of byte j + 4 with the top two bits of bytes j - 4 and j.
function subBlockScaleMin(s, o, j) {
  if (j < 4) return [s[o + j] & 63, s[o + j + 4] & 63];
  return [(s[o + j + 4] & 15) | ((s[o + j - 4] >> 6) << 4), (s[o + j + 4] >> 4) | ((s[o + j] >> 6) << 4)];
}

// One 144-byte block at w[o..] -> 256 values into row[r..r+255]. Group g of
// 32 bytes holds sub-block 2g in its low nibbles, 2g + 1 in its high ones.
function decodeBlock(w, o, row, r) {
  const d = halfBitsToNumber(w[o] | (w[o + 1] << 8));
  const dmin = halfBitsToNumber(w[o + 2] | (w[o + 3] << 8));
  for (let g = 0; g < 4; g += 1) {
    const lo = subBlockScaleMin(w, o + 4, 2 * g);
    const hi = subBlockScaleMin(w, o + 4, 2 * g + 1);
    const q = o + 16 + 32 * g;
    const out = r + 64 * g;
    for (let i = 0; i < 32; i += 1) {
      const b = w[q + i];
      row[out + i] = d * lo[0] * (b & 15) - dmin * lo[1];
      row[out + 32 + i] = d * hi[0] * (b >> 4) - dmin * hi[1];
    }
  }
}

function matmul(w, x, m, n, k, y) {
  const blocks = k / 256;
  const row = new Float32Array(k);
  for (let j = 0; j < n; j += 1) {
    for (let b = 0; b < blocks; b += 1) decodeBlock(w, (j * blocks + b) * 144, row, 256 * b);
    for (let i = 0; i < m; i += 1) {
      let acc = 0;
      const xo = i * k;
      for (let t = 0; t < k; t += 1) acc += x[xo + t] * row[t];
      y[i * n + j] = acc;
    }
  }
}

function main(argv) {
  const [wPath, xPath, ms, ns, ks, runsArg, yPath] = argv;
  const m = Number(ms), n = Number(ns), k = Number(ks), runs = Math.max(1, Number(runsArg));
  if (!(k % 256 === 0 && m > 0 && n > 0)) throw new Error('k must be a multiple of 256');
  const w = new Uint8Array(fs.readFileSync(wPath));
  if (w.length !== n * (k / 256) * 144) throw new Error(`W has ${w.length} bytes; expected ${n * (k / 256) * 144}`);
  const xb = fs.readFileSync(xPath);
  const x = new Float32Array(m * k);
  for (let i = 0; i < m * k; i += 1) x[i] = halfBitsToNumber(xb[2 * i] | (xb[2 * i + 1] << 8));
  const y = new Float64Array(m * n);
  matmul(w, x, m, n, k, y); // warm-up
  const times = [];
  for (let r = 0; r < runs; r += 1) {
    const t0 = process.hrtime.bigint();
    matmul(w, x, m, n, k, y);
    times.push(Number(process.hrtime.bigint() - t0) / 1e6);
  }
  const sorted = times.slice().sort((a, b) => a - b);
  let checksum = 0;
  for (let i = 0; i < y.length; i += 1) checksum += y[i];
  if (yPath) fs.writeFileSync(yPath, Buffer.from(y.buffer));
  console.log(JSON.stringify({ ms: times, ms_median: sorted[Math.floor(sorted.length / 2)], node: process.version,
    checksum }));
}

main(process.argv.slice(2));
