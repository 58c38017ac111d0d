'use strict';
// The JS host without a GPU: the pack format (tests/prepacked-format.test.ts:13-33
// re-expressed, parser errors), the addon's exports and argument checks.
// With an output path argument it also writes a pack built from fixed inputs
// so the Python test can compare it byte for byte with its own builder.
const assert = require('assert');
const fs = require('fs');
const path = require('path');
const { test, run } = require('./harness');
const host = require(path.join(__dirname, '..', '..', 'nemotron-3-embed-webgpu_amd', 'js'));

function q40Block(scaleBits, quants) {
  const block = new Uint8Array(18);
  block.set(scaleBits, 0);
  for (let i = 0; i < 16; i += 1) block[i + 2] = quants[i] | (quants[i + 16] << 4);
  return block;
}

function referencePack() {
  const first = q40Block([0x00, 0x3c], Array.from({ length: 32 }, (_, i) => i & 15));
  const second = q40Block([0x00, 0x40], Array.from({ length: 32 }, (_, i) => 15 - (i & 15)));
  const packed = host.packQ40Tile32('fused', [{ name: 'first', k: 32, n: 1, bytes: first }, { name: 'second', k: 32, n: 1, bytes: second }]);
  const raw = host.rawTensor('norm', [1], host.GGMLType.F32, new Uint8Array([1, 2, 3, 4]));
  return { packed, file: host.buildPrepackedFile('abc123', 42, { 'general.name': 'test' }, [raw, packed]) };
}

test('builds and parses the reference pack', () => {
  const { packed, file } = referencePack();
  assert.deepStrictEqual(packed.dimensions, [32, 2]);
  assert.strictEqual(packed.bytes.byteLength, 32 * 20);
  assert.deepStrictEqual(Array.from(packed.bytes.slice(0, 8)), [0x00, 0x3c, 0x00, 0x00, 0x00, 0x11, 0x22, 0x33]);
  assert.deepStrictEqual(Array.from(packed.bytes.slice(20, 28)), [0x00, 0x40, 0x00, 0x00, 0xff, 0xee, 0xdd, 0xcc]);
  const parsed = host.parsePrepackedModel(file.buffer);
  assert.strictEqual(parsed.header.sourceSha256, 'abc123');
  assert.strictEqual(parsed.header.sourceBytes, 42);
  assert.strictEqual(parsed.header.metadata['general.name'], 'test');
  const norm = parsed.tensors.get('norm');
  assert.deepStrictEqual([norm.dimensions, norm.type, norm.storage, norm.byteLength], [[1], 0, 'raw', 4]);
  const fused = parsed.tensors.get('fused');
  assert.deepStrictEqual([fused.dimensions, fused.type, fused.storage, fused.byteLength], [[32, 2], 2, 'q4_0-tile32-compact', 640]);
  assert.strictEqual(parsed.dataOffset % 256, 0);
});

test('parser errors match the reference messages', () => {
  const { file } = referencePack();
  assert.throws(() => host.parsePrepackedModel(new ArrayBuffer(4)), /shorter than its prelude/);
  const badMagic = file.slice();
  badMagic[7] = 0x31;
  assert.throws(() => host.parsePrepackedModel(badMagic.buffer), /invalid prepacked model magic "WGPACK01"/);
  const truncated = file.slice(0, file.byteLength - 1);
  assert.throws(() => host.parsePrepackedModel(truncated.buffer), /fused extends past end of prepacked file/);
  const longHeader = file.slice();
  new DataView(longHeader.buffer).setUint32(8, 1 << 30, true);
  assert.throws(() => host.parsePrepackedModel(longHeader.buffer), /header extends past end of file/);
});

test('addon exports the C ABI surface and checks its arguments', () => {
  const n = host.native();
  for (const name of ['version', 'dimsReference', 'profileStageNames', 'init', 'shutdown', 'modelCreate', 'modelSetTensor',
    'modelSynthesize', 'modelFinalize', 'modelDestroy', 'planCreate', 'planRun', 'planProfile', 'planDestroy']) {
    assert.strictEqual(typeof n[name], 'function', name);
  }
  assert.ok(n.version().startsWith('libnemo'));
  const d = host.referenceDims();
  assert.deepStrictEqual([d.hidden, d.qHeads, d.kvHeads, d.headDim, d.intermediate, d.layers, d.vocab, d.mergeAfterLayer],
    [2048, 24, 8, 128, 6144, 16, 131072, 4]);
  assert.deepStrictEqual(n.profileStageNames(), ['embedding_norm', 'token_merge', 'qkv', 'rope_attention', 'attention_output',
    'post_attention_norm', 'ffn_up_gate', 'swiglu', 'ffn_down', 'post_ffn_norm', 'pool']);
  assert.throws(() => n.planRun({}, new Uint32Array(1), new Uint32Array(1), 1), /expected a plan handle/);
  assert.throws(() => n.modelCreate(1), /wrong number of arguments/);
  assert.strictEqual(host.contextualMergedLength(150), 96);
  assert.strictEqual(host.contextualMergedLength(5000), 3200);
});

if (process.argv[2]) {
  const n = 40;
  const k = 64;
  const raw = new Uint8Array(n * (k / 32) * 18);
  for (let i = 0; i < raw.length; i += 1) raw[i] = (i * 37 + 11) & 255;
  const packed = host.packQ40Tile32('m', [{ name: 'a', k, n: 10, bytes: raw.subarray(0, 10 * 2 * 18) },
    { name: 'b', k, n: 30, bytes: raw.subarray(10 * 2 * 18) }]);
  const norm = host.rawTensor('norm', [4], 0, new Uint8Array(16).fill(7));
  fs.writeFileSync(process.argv[2], host.buildPrepackedFile('feed', 123, { 'general.name': 'cross' }, [norm, packed]));
}

run();
