'use strict';
/*
 * Loader of the q8hip N-API addon (built next to this file by
 * `python -m mlfw_amd.build`).  There is no fallback: a missing or
 * unloadable addon is an error, never a silent CPU path.
 */
const path = require('path');

const ADDON = path.join(__dirname, 'q8hip.node');

let addon;
try {
  addon = require(ADDON);
} catch (err) {
  const e = new Error(`q8hip addon not loadable from ${ADDON}: ${err.message} ` +
                      '(build it with `python -m mlfw_amd.build`; there is no CPU fallback)');
  e.cause = err;
  throw e;
}

module.exports = addon;
