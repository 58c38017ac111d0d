'use strict';
// The JS host on an MI355X: node tests/js/gpu.test.js <model.wgpack> <tiny_forward.json>
// The pack holds the tiny golden model's raw Q4_K/Q6_K/F16/F32 tensors; the
// embeddings must match the oracle's frozen values (cosine >= 0.9999).
const assert = require('assert');
const fs = require('fs');
const path = require('path');
const { test, run } = require('./harness');
const host = require(path.join(__dirname, '..', '..', 'nemotron-3-embed-webgpu_amd', 'js'));

const [packPath, goldenPath] = process.argv.slice(2);
const golden = JSON.parse(fs.readFileSync(goldenPath, 'utf8'));
const g = golden.dims;
const dims = {
  hidden: g.hidden, qHeads: g.q_heads, kvHeads: g.kv_heads, headDim: g.head_dim, intermediate: g.intermediate,
  layers: g.layers, vocab: g.vocab, mergeAfterLayer: g.merge_after_layer, kvStrideThreshold: g.kv_stride_threshold,
};
const expected = golden.embeddings_f32_bits.map((bits) => new Float32Array(Uint32Array.from(bits).buffer));

function cosine(a, b) {
  let ab = 0;
  let aa = 0;
  let bb = 0;
  for (let i = 0; i < a.length; i += 1) { ab += a[i] * b[i]; aa += a[i] * a[i]; bb += b[i] * b[i]; }
  return ab / Math.sqrt(aa * bb);
}

function norm(a) {
  let s = 0;
  for (let i = 0; i < a.length; i += 1) s += a[i] * a[i];
  return Math.sqrt(s);
}

const device = host.requestHipDevice(0);
const file = fs.readFileSync(packPath);
const pack = host.parsePrepackedModel(file.buffer.slice(file.byteOffset, file.byteOffset + file.byteLength));
const model = new host.NemotronHipModel(device, pack, { dims });
const tokenizer = (text) => ({ input_ids: { tolist: () => [text.split(',').map(Number)] } });

test('engine embeddings match the golden fixture', async () => {
  const created = [];
  const plans = [];
  const runtime = {
    maxStorageBufferBindingSize: model.maxStorageBufferBindingSize,
    createPlan(batch, sequence) {
      created.push([batch, sequence]);
      const plan = model.createPlan(batch, sequence);
      plans.push(plan);
      return plan;
    },
  };
  const engine = new host.NemotronEmbeddingEngine(runtime, tokenizer);
  const out = await Promise.all(golden.requests.map((r) => engine.embed(r.join(','))));
  const longest = Math.max.apply(null, golden.requests.map((r) => r.length));
  assert.deepStrictEqual(created, [[golden.requests.length, longest]]);
  out.forEach((e, i) => {
    assert.ok(e instanceof Float32Array && e.length === dims.hidden);
    const c = cosine(e, expected[i]);
    assert.ok(c >= 0.9999, `request ${i}: cosine ${c}`);
    assert.ok(Math.abs(norm(e) - 1) <= 0.01);
  });
  plans.forEach((p) => p.destroy());
});

test('plan errors and profile mirror the reference', async () => {
  const plan = model.createPlan(2, 8);
  await assert.rejects(plan.run(new Uint32Array(15), new Uint32Array([8, 8])), /token buffer does not match execution plan/);
  const ids = new Uint32Array(16).fill(3);
  ids[0] = 1;
  ids[8] = 1;
  const stages = await plan.profile(ids, new Uint32Array([8, 5]));
  assert.deepStrictEqual(Object.keys(stages), host.native().profileStageNames());
  assert.ok(Object.values(stages).every((ms) => ms >= 0) && stages.ffn_up_gate > 0);
  plan.destroy();
  await assert.rejects(plan.profile(ids, new Uint32Array([8, 5])), /plan was destroyed/);
  await assert.rejects(plan.run(ids, new Uint32Array([8, 5])), /plan was destroyed/);
});

test('distinct plans run concurrently and agree with single runs', async () => {
  const reqs = golden.requests;
  const singles = reqs.map((r) => model.createPlan(1, r.length));
  const outs = await Promise.all(singles.map((p, i) => p.run(Uint32Array.from(reqs[i]), new Uint32Array([reqs[i].length]))));
  outs.forEach((o, i) => {
    assert.ok(cosine(o[0], expected[i]) >= 0.9999);
  });
  singles.forEach((p) => p.destroy());
});

test('destroy while runs are pending: the runs resolve, the plan is freed after them', async () => {
  const reqs = golden.requests;
  const longest = Math.max.apply(null, reqs.map((r) => r.length));
  const ids = new Uint32Array(reqs.length * longest).fill(11);
  reqs.forEach((r, i) => ids.set(r, i * longest));
  const lengths = Uint32Array.from(reqs.map((r) => r.length));
  const plan = model.createPlan(reqs.length, longest);
  const first = plan.run(ids, lengths);
  const second = plan.run(ids, lengths);
  plan.destroy();
  await assert.rejects(plan.run(ids, lengths), /plan was destroyed/);
  const [a, b] = await Promise.all([first, second]);
  [a, b].forEach((out) => out.forEach((e, i) => assert.ok(cosine(e, expected[i]) >= 0.9999, `request ${i}`)));
  assert.strictEqual(plan.pending, 0);
  assert.ok(plan.destroyed);
  // the addon's own guard: a direct planDestroy with a run in flight also defers
  const raw = host.native().planCreate(model.handle, reqs.length, longest);
  const inFlight = host.native().planRun(raw, ids, lengths);
  host.native().planDestroy(raw);
  assert.throws(() => host.native().planRun(raw, ids, lengths), /plan was destroyed/);
  const out = await inFlight;
  assert.strictEqual(out.length, reqs.length * dims.hidden);
});

test('synthetic config-dims model: 16 concurrent 150-token requests, one plan run', async () => {
  const cfg = Object.assign(host.configDims(), { layers: 2, mergeAfterLayer: 1 });
  const synth = new host.NemotronHipModel(device, { synthetic: 1003 }, { dims: cfg });
  let runs = 0;
  const plans = [];
  const runtime = {
    createPlan(batch, sequence) {
      const plan = synth.createPlan(batch, sequence);
      plans.push(plan);
      return { run(ids, lengths) { runs += 1; return plan.run(ids, lengths); } };
    },
  };
  const engine = new host.NemotronEmbeddingEngine(runtime, tokenizer);
  const texts = Array.from({ length: 16 }, (_, r) => Array.from({ length: 149 }, (_, t) => 2 + ((r * 7919 + t * 104729) % 131000)).join(','));
  const t0 = Date.now();
  const out = await Promise.all(texts.map((t) => engine.embed(t)));
  console.log(`  16 x 150 tokens, 2 layers: ${Date.now() - t0} ms including plan creation`);
  assert.strictEqual(runs, 1);
  out.forEach((e) => assert.ok(Math.abs(norm(e) - 1) <= 0.01));
  plans.forEach((p) => p.destroy());
  synth.destroy();
});

run().then(() => {
  model.destroy();
  device.destroy();
});
