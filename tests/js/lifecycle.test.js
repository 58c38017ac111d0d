'use strict';
// Plan lifetime in the JS host without a GPU: NemotronHipPlan against a
// stand-in for the addon that records calls and holds each run until the
// test settles it. destroy() while a run is pending must close the plan to
// new calls at once, let the pending run resolve, and free the native plan
// exactly once, after it (src/webgpu/model.ts:141-144).
const assert = require('assert');
const path = require('path');
const { test, run } = require('./harness');

const JS = path.join(__dirname, '..', '..', 'nemotron-3-embed-webgpu_amd', 'js');
const calls = [];
let settlers = [];
const fake = {
  dimsReference: () => ({ hidden: 4, qHeads: 2, kvHeads: 1, headDim: 64, intermediate: 256, layers: 1, vocab: 8 }),
  modelCreate: () => ({ model: true }),
  modelSynthesize: () => {},
  modelFinalize: () => {},
  modelDestroy: () => calls.push('modelDestroy'),
  planCreate: () => ({ plan: true }),
  planRun: (handle, ids, lengths) => {
    calls.push('planRun');
    return new Promise((resolve, reject) => settlers.push({ resolve, reject, batch: lengths.length }));
  },
  planProfile: () => ({}),
  planDestroy: () => calls.push('planDestroy'),
};
const nativePath = require.resolve(path.join(JS, 'native.js'));
require.cache[nativePath] = { id: nativePath, filename: nativePath, loaded: true, exports: { native: () => fake } };
const { NemotronHipModel } = require(path.join(JS, 'runtime.js'));

function newPlan(batch) {
  calls.length = 0;
  settlers = [];
  const model = new NemotronHipModel({ handle: 1 }, { synthetic: 1 });
  return model.createPlan(batch, 3);
}

test('destroy while a run is pending frees the plan after the run resolves', async () => {
  const plan = newPlan(2);
  const pending = plan.run([1, 2, 3, 1, 2, 11], [3, 2]);
  plan.destroy();
  assert.deepStrictEqual(calls, ['planRun']);
  await assert.rejects(plan.run([1, 2, 3, 1, 2, 11], [3, 2]), /plan was destroyed/);
  await assert.rejects(plan.profile([1, 2, 3, 1, 2, 11], [3, 2]), /plan was destroyed/);
  settlers[0].resolve(new Float32Array(2 * 4).fill(0.5));
  const out = await pending;
  assert.strictEqual(out.length, 2);
  assert.strictEqual(out[0].length, 4);
  assert.deepStrictEqual(calls, ['planRun', 'planDestroy']);
  plan.destroy();
  assert.deepStrictEqual(calls, ['planRun', 'planDestroy']);
});

test('the last of several pending runs frees the plan', async () => {
  const plan = newPlan(1);
  const a = plan.run([1, 2, 3], [3]);
  const b = plan.run([1, 2, 11], [2]);
  plan.destroy();
  settlers[1].resolve(new Float32Array(4));
  await b;
  assert.deepStrictEqual(calls, ['planRun', 'planRun']);
  settlers[0].resolve(new Float32Array(4));
  await a;
  assert.deepStrictEqual(calls, ['planRun', 'planRun', 'planDestroy']);
});

test('a failed run settles the count', async () => {
  const plan = newPlan(1);
  const pending = plan.run([1, 2, 3], [3]);
  plan.destroy();
  settlers[0].reject(new Error('device lost'));
  await assert.rejects(pending, /device lost/);
  assert.deepStrictEqual(calls, ['planRun', 'planDestroy']);
});

test('destroy without runs frees at once', async () => {
  const plan = newPlan(1);
  plan.destroy();
  assert.deepStrictEqual(calls, ['planDestroy']);
  await assert.rejects(plan.run([1, 2, 3], [3]), /plan was destroyed/);
});

run();
