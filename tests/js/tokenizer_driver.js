'use strict';
// Runs Gemma4Tokenizer over a batch of requests.
// argv: tokenizer directory, requests.json
// requests: {encode: [text], decode: [[id]], decodeRaw: [[id]], decodeTokens: [[token]],
//            chat: [{messages, opts}], badChat: [messages], stop: bool, describe: bool,
//            split: [[raw, plain]]}
// Prints one JSON line with the results under the same keys.
const fs = require('fs');
const { Gemma4Tokenizer } = require('../../gemma4-js_amd/node/tokenizer.js');
const { splitReasoningOutput } = require('../../gemma4-js_amd/node/generate.js');

const tk = Gemma4Tokenizer.fromDirectorySync(process.argv[2]);
const req = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
const out = {};
if (req.encode) out.encode = req.encode.map((t) => tk.encode(t));
if (req.decode) out.decode = req.decode.map((ids) => tk.decode(ids));
if (req.decodeRaw) out.decodeRaw = req.decodeRaw.map((ids) => tk.decode(ids, { skipSpecialTokens: false }));
if (req.decodeTokens) out.decodeTokens = req.decodeTokens.map((toks) => tk.decodeTokens(toks));
if (req.chat) out.chat = req.chat.map((c) => tk.encodeChat(c.messages, c.opts));
if (req.badChat) {
  out.badChat = req.badChat.map((m) => {
    try { tk.renderChat(m); return null; } catch (e) { return e.message; }
  });
}
if (req.stop) out.stop = Array.from(tk.stopTokenIds()).sort((a, b) => a - b);
if (req.describe) out.describe = tk.describe();
if (req.split) out.split = req.split.map((p) => splitReasoningOutput(p[0], p[1]));
console.log(JSON.stringify(out));
