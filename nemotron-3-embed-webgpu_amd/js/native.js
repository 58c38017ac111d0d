'use strict';
// Loads the Node-API addon (nemo_napi.node, built by napi/Makefile next to
// libnemo.so). There is no fallback: without the addon every use throws.
const path = require('path');

const ADDON_PATH = path.join(__dirname, '..', 'nemo_napi.node');
let addon = null;

function native() {
  if (addon === null) {
    try {
      addon = require(ADDON_PATH);
    } catch (error) {
      const wrapped = new Error(`nemo_napi.node could not be loaded from ${ADDON_PATH}: ${error.message}`);
      wrapped.cause = error;
      throw wrapped;
    }
  }
  return addon;
}

module.exports = { native, ADDON_PATH };
