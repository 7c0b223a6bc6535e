'use strict';
// The text generation loop of the reference's page (custom-webgpu/main.js:342-556)
// as a library function for Node.
//
// One user message is rendered with the Gemma 4 chat template and encoded.
// The prompt is prefilled with model.greedy(ids, 0). Then, as in main.js:
//   - a stop token (generation_config eos ids, <eos>, <turn|>) ends the loop
//     before it is appended;
//   - otherwise the token is appended and the text is re-decoded;
//   - the loop ends at maxNewTokens, or when the next position would reach
//     the KV-cache capacity maxSeq;
//   - else the token is fed at position prompt + generated - 1.
//
// `chunk` selects how the next tokens are computed:
//   0 (default): one model.greedy([token], position) per token, as main.js does;
//   n > 0: model.decode(k) with k <= n, the device-side decode loop of
//          Gemma4HipEngine (one graph replay per token, no logits read back).
// Both give the same tokens. A chunk can run past a stop token; the
// generated list ends at the stop token all the same, but the KV cache then
// holds up to n - 1 tokens more than the one-token loop would leave.

const THOUGHT_START = '<|channel>thought\n';
const CHANNEL_END = '<channel|>';

// Reasoning and answer of a Gemma 4 output (main.js:127-161): the text between
// "<|channel>thought\n" and "<channel|>" is the reasoning; what follows, minus
// a leading "<|channel>final\n", a trailing "<channel|>" and leading
// whitespace, is the answer (the plain text when that is empty).
function splitReasoningOutput(rawText, plainText) {
  const at = rawText.indexOf(THOUGHT_START);
  if (at < 0) return { reasoning: '', answer: plainText };
  const bodyStart = at + THOUGHT_START.length;
  const end = rawText.indexOf(CHANNEL_END, bodyStart);
  if (end < 0) return { reasoning: rawText.slice(bodyStart), answer: '' };
  const answer = rawText.slice(end + CHANNEL_END.length)
    .replace(/^<\|channel>final\n/u, '')
    .replace(/<channel\|>$/u, '')
    .trimStart();
  return { reasoning: rawText.slice(bodyStart, end), answer: answer || plainText };
}

function now() { return Number(process.hrtime.bigint()) / 1e6; }

// model: the Gemma4WebGPU surface (resetCache, greedy; decode for chunk > 0).
// tokenizer: a Gemma4Tokenizer.
// opts: maxNewTokens (default 128), maxSeq (required: the model's KV-cache
// capacity), enableThinking, chunk, onToken({step, id, text, reasoning,
// answer}) called after each appended token (return true to stop),
// shouldStop() polled before each token (the page's Stop button).
async function generate(model, tokenizer, prompt, opts) {
  opts = opts || {};
  const maxNewTokens = opts.maxNewTokens === undefined ? 128 : Number(opts.maxNewTokens);
  const maxSeq = Number(opts.maxSeq);
  if (!(maxSeq > 0)) throw new Error('generate: maxSeq (the KV-cache capacity) is required');
  const chunk = opts.chunk ? Number(opts.chunk) : 0;
  if (chunk > 0 && typeof model.decode !== 'function') throw new Error('generate: chunk > 0 needs model.decode');

  model.resetCache();
  const enc = tokenizer.encodeChat([{ role: 'user', content: prompt }],
    { addGenerationPrompt: true, enableThinking: Boolean(opts.enableThinking) });
  const inputIds = enc.ids;
  if (inputIds.length >= maxSeq) {
    throw new Error(`Prompt length ${inputIds.length} exceeds KV-cache capacity ${maxSeq}.`);
  }
  const stopIds = tokenizer.stopTokenIds();
  const generated = [];
  const decodeTimes = [];
  let stopReason = 'max_new_tokens';
  let stopTokenId = null;

  let t0 = now();
  let nextId = (await model.greedy(inputIds, 0)).nextTokenId;
  const prefillMs = now() - t0;

  let ahead = [];  // tokens already computed by model.decode
  for (let step = 0; step < maxNewTokens; step++) {
    if (opts.shouldStop && opts.shouldStop()) { stopReason = 'stopped'; break; }
    if (stopIds.has(nextId)) { stopReason = 'stop_token'; stopTokenId = nextId; break; }
    generated.push(nextId);
    if (opts.onToken) {
      const text = tokenizer.decode(generated, { skipSpecialTokens: true });
      const raw = tokenizer.decode(generated, { skipSpecialTokens: false });
      const sep = splitReasoningOutput(raw, text);
      if (opts.onToken({ step, id: nextId, text, reasoning: sep.reasoning, answer: sep.answer }) === true) {
        stopReason = 'stopped';
        break;
      }
    }
    if (generated.length >= maxNewTokens) break;
    const position = inputIds.length + generated.length - 1;
    if (position >= maxSeq) { stopReason = 'kv_capacity'; break; }
    t0 = now();
    if (chunk > 0) {
      if (ahead.length === 0) {
        // never past maxNewTokens, never past the cache capacity
        const k = Math.min(chunk, maxNewTokens - generated.length, maxSeq - position);
        ahead = Array.from(model.decode(k));
      }
      nextId = ahead.shift();
    } else {
      nextId = (await model.greedy([nextId], position)).nextTokenId;
    }
    decodeTimes.push(now() - t0);
  }

  const text = tokenizer.decode(generated, { skipSpecialTokens: true });
  const rawText = tokenizer.decode(generated, { skipSpecialTokens: false });
  const sep = splitReasoningOutput(rawText, text);
  const decodeMs = decodeTimes.reduce((a, b) => a + b, 0);
  return {
    rendered: enc.rendered, inputIds, generated, text, rawText,
    reasoning: sep.reasoning, answer: sep.answer, stopReason, stopTokenId,
    prefillMs, decodeMs, msPerToken: decodeTimes.length ? decodeMs / decodeTimes.length : null,
  };
}

module.exports = { generate, splitReasoningOutput };
