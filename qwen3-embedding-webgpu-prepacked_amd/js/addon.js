'use strict';
// Loads the N-API addon built next to this file (js/build/qattn_napi.node, which links
// ../libqattn.so).  There is no fallback: a missing addon or library is an error.
const path = require('path');

let cached = null;

function loadAddon() {
  if (cached) return cached;
  const file = path.join(__dirname, 'build', 'qattn_napi.node');
  try {
    cached = require(file);
  } catch (error) {
    throw new Error(`qattn N-API addon not loadable from ${file} (build it with make -C the package directory): ${error.message}`);
  }
  return cached;
}

module.exports = { loadAddon };
