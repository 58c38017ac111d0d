'use strict';
// NemotronEmbeddingEngine (JS host) with fake runtimes, as the reference's own
// tests drive it (tests/embedding-engine.test.ts:5-50), plus the failure path.
const assert = require('assert');
const path = require('path');
const { test, run } = require('./harness');
const { NemotronEmbeddingEngine } = require(path.join(__dirname, '..', '..', 'nemotron-3-embed-webgpu_amd', 'js', 'engine'));

test('coalesces up to 16 simultaneous requests and preserves result order', async () => {
  const calls = [];
  const runtime = {
    createPlan(batch, sequence) {
      return {
        async run(ids, lengths) {
          calls.push({ batch, sequence, ids: Array.from(ids), lengths: Array.from(lengths) });
          return Array.from({ length: batch }, (_, i) => new Float32Array([ids[i * sequence + 1]]));
        },
      };
    },
  };
  const tokenizer = (text) => ({ input_ids: { tolist: () => [[Number(text)]] } });
  const engine = new NemotronEmbeddingEngine(runtime, tokenizer, 16, 0, 99);
  const results = await Promise.all(Array.from({ length: 16 }, (_, i) => engine.embed(String(i + 1))));
  assert.strictEqual(calls.length, 1);
  assert.strictEqual(calls[0].batch, 16);
  assert.strictEqual(calls[0].sequence, 2);
  assert.deepStrictEqual(calls[0].lengths, Array(16).fill(2));
  assert.deepStrictEqual(results.map((v) => v[0]), Array.from({ length: 16 }, (_, i) => i + 1));
});

test('pads mixed-length requests after their final token', async () => {
  let recorded = [];
  const runtime = {
    createPlan(batch) {
      return { async run(ids) { recorded = Array.from(ids); return Array.from({ length: batch }, () => new Float32Array(1)); } };
    },
  };
  const tokenizer = (text) => ({ input_ids: { tolist: () => [text.split(',').map(Number)] } });
  const engine = new NemotronEmbeddingEngine(runtime, tokenizer, 16, 0, 99, 99);
  await Promise.all([engine.embed('1'), engine.embed('2,3')]);
  assert.deepStrictEqual(recorded, [99, 1, 99, 99, 2, 3]);
});

test('splits batches to stay within the storage-binding limit', async () => {
  const batches = [];
  const runtime = {
    maxStorageBufferBindingSize: 2 * 6144 * 2 * 2,
    createPlan(batch) {
      return { async run() { batches.push(batch); return Array.from({ length: batch }, () => new Float32Array(1)); } };
    },
  };
  const engine = new NemotronEmbeddingEngine(runtime, () => ({ input_ids: { tolist: () => [[1]] } }), 16, 0, 1);
  await Promise.all(Array.from({ length: 5 }, () => engine.embed('x')));
  assert.deepStrictEqual(batches, [2, 2, 1]);
});

test('caps long sequences at 8 per batch and caches plans', async () => {
  const created = [];
  const runs = [];
  const runtime = {
    createPlan(batch, sequence) {
      created.push([batch, sequence]);
      return { async run() { runs.push(batch); return Array.from({ length: batch }, () => new Float32Array(1)); } };
    },
  };
  const engine = new NemotronEmbeddingEngine(runtime, () => ({ input_ids: { tolist: () => [Array(1500).fill(1)] } }), 16, 0, 1);
  await Promise.all(Array.from({ length: 16 }, () => engine.embed('x')));
  assert.deepStrictEqual(runs, [8, 8]);
  assert.deepStrictEqual(created, [[8, 1500]]);
});

test('a failing run rejects its whole batch and the queue drains', async () => {
  const runs = [];
  const runtime = {
    createPlan(batch) {
      return {
        async run() {
          runs.push(batch);
          if (runs.length === 1) throw new Error('device lost');
          return Array.from({ length: batch }, (_, i) => new Float32Array([i]));
        },
      };
    },
  };
  const tokenizer = (text) => ({ input_ids: { tolist: () => [[1, Number(text)]] } });
  const engine = new NemotronEmbeddingEngine(runtime, tokenizer, 2, 0, 1);
  const settled = await Promise.all(Array.from({ length: 5 }, (_, i) => engine.embed(String(i)).then((v) => v[0], (e) => e.message)));
  assert.deepStrictEqual(runs, [2, 2, 1]);
  assert.deepStrictEqual(settled, ['device lost', 'device lost', 0, 1, 0]);
});

test('rejects batch sizes outside 1..16', () => {
  for (const bad of [0, 17]) assert.throws(() => new NemotronEmbeddingEngine({}, () => null, bad), /maxBatchSize must be between 1 and 16/);
});

run();
