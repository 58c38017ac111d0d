'use strict';
// Minimal sequential test runner for the Node tests (no framework is
// installed): test(name, fn) registers, run() executes in order, prints
// "ok"/"not ok" lines and exits non-zero on any failure.
const tests = [];

function test(name, fn) {
  tests.push({ name, fn });
}

async function run() {
  let failed = 0;
  for (const t of tests) {
    try {
      await t.fn();
      console.log(`ok - ${t.name}`);
    } catch (error) {
      failed += 1;
      console.log(`not ok - ${t.name}\n  ${error && error.stack ? error.stack : error}`);
    }
  }
  console.log(`${tests.length - failed}/${tests.length} passed`);
  process.exitCode = failed ? 1 : 0;
}

module.exports = { test, run };
