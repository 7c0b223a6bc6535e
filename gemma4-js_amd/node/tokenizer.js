'use strict';
// Gemma 4 text tokenizer for Node: the host-side counterpart of the reference's
// Gemma4Tokenizer (custom-webgpu/standalone-tokenizer.js:294-827), written for
// Node 12 (no `?.`, `??` or String#replaceAll).
//
// It reads a Hugging Face tokenizer.json whose model is BPE. The Gemma 4 file
// is: normalizer Replace(" " -> "▁"), pre-tokenizer Split(" ",
// MergedWithPrevious) (a no-op once the spaces are replaced), BPE with
// byte_fallback over 262144 tokens and 514906 merges, and decoder
// Replace("▁" -> " "), ByteFallback, Fuse.
//
// Encoding (standalone-tokenizer.js:405-598):
//   normalize -> split out special added tokens -> pre-tokenize -> BPE each piece.
// BPE (484-572): the piece starts as its code points; a code point missing
// from the vocabulary becomes its UTF-8 byte tokens <0xHH>. Then, while any
// adjacent pair has a merge rule, the pair with the lowest rank is merged, the
// leftmost one among equal ranks. Here the candidate pairs sit in a binary
// heap ordered by (rank, position), so a piece of n symbols costs
// O(n log n) instead of the reference's rescan of every pair per merge; the
// merge chosen at each step is the same.

const fs = require('fs');
const path = require('path');

const UTF8_ENCODER = new TextEncoder();
const UTF8_DECODER = new TextDecoder('utf-8', { fatal: false });

function def(v, d) { return v === undefined || v === null ? d : v; }
function replaceEvery(text, from, to) { return from === '' ? text : text.split(from).join(to); }
function escapeRegex(s) { return s.replace(/[.*+?^${}()|[\]\\]/g, '\\$&'); }

// A Split/Replace pattern is {Regex: source} or {String: literal} (standalone-tokenizer.js:10-28).
function regexSource(pattern) {
  if (typeof pattern === 'string') return pattern;
  if (pattern && typeof pattern === 'object') {
    if (typeof pattern.Regex === 'string') return pattern.Regex;
    if (typeof pattern.String === 'string') return escapeRegex(pattern.String);
  }
  throw new Error(`Unsupported Split pattern: ${JSON.stringify(pattern)}`);
}

function byteToken(b) { return '<0x' + b.toString(16).toUpperCase().padStart(2, '0') + '>'; }

function parseByteToken(token) {
  const m = /^<0x([0-9A-Fa-f]{2})>$/.exec(token);
  return m ? parseInt(m[1], 16) : null;
}

// Sequence nodes are flattened; their children sit under `decoders`,
// `pretokenizers` or `pre_tokenizers`.
function flatten(node, key, altKey) {
  if (!node) return [];
  if (node.type !== 'Sequence') return [node];
  const kids = def(node[key], def(altKey ? node[altKey] : undefined, []));
  const out = [];
  for (const k of kids) out.push(...flatten(k, key, altKey));
  return out;
}

function normalize(text, n) {
  if (!n) return text;
  switch (n.type) {
    case 'Sequence':
      return def(n.normalizers, []).reduce((t, m) => normalize(t, m), text);
    case 'NFC': case 'NFD': case 'NFKC': case 'NFKD':
      return text.normalize(n.type);
    case 'Lowercase':
      return text.toLowerCase();
    case 'Replace':
      return text.replace(new RegExp(regexSource(n.pattern), 'gu'), def(n.content, ''));
    case 'Prepend':
      return def(n.prepend, '') + text;
    case 'Precompiled':
      throw new Error('Precompiled tokenizer normalizer is not supported by the standalone runtime.');
    default:
      throw new Error(`Unsupported normalizer: ${n.type}`);
  }
}

// A part is {text, special}; special parts pass through every pre-tokenizer.

// Split (standalone-tokenizer.js:75-170): matched and unmatched stretches
// become parts; `behavior` decides what happens to the matched ones.
function splitParts(parts, cfg) {
  const re = new RegExp(regexSource(cfg.pattern), 'gu');
  const behavior = def(cfg.behavior, 'Isolated');
  const invert = Boolean(cfg.invert);
  const out = [];
  const emit = (value, isMatch) => {
    if (value.length === 0) return;
    if (!(invert ? !isMatch : isMatch)) { out.push({ text: value, special: false }); return; }
    if (behavior === 'Removed') return;
    const last = out[out.length - 1];
    if (behavior === 'MergedWithPrevious' && last && !last.special) { last.text += value; return; }
    if (behavior === 'MergedWithNext') { out.push({ text: value, special: false, mergeNext: true }); return; }
    out.push({ text: value, special: false });
  };
  for (const part of parts) {
    if (part.special) { out.push(part); continue; }
    const text = part.text;
    let cursor = 0;
    for (const m of Array.from(text.matchAll(re))) {
      const at = def(m.index, 0);
      emit(text.slice(cursor, at), false);
      emit(m[0], true);
      cursor = at + m[0].length;
    }
    emit(text.slice(cursor), false);
  }
  // a MergedWithNext part is joined to whatever part follows it
  const merged = [];
  for (const p of out) {
    const last = merged[merged.length - 1];
    if (last && last.mergeNext) { merged[merged.length - 1] = { text: last.text + p.text, special: false }; continue; }
    merged.push(p);
  }
  return merged;
}

// Metaspace (standalone-tokenizer.js:172-229). As in the reference, the
// prepend scheme is "always" whenever prepend_scheme (or, without it,
// add_prefix_space) is truthy, and "never" otherwise.
function metaspaceParts(parts, cfg) {
  const rep = def(cfg.replacement, '▁');
  const scheme = def(cfg.prepend_scheme, cfg.add_prefix_space) ? 'always' : 'never';
  const split = def(cfg.split, true);
  const out = [];
  parts.forEach((part, index) => {
    if (part.special) { out.push(part); return; }
    let text = replaceEvery(part.text, ' ', rep);
    const prepend = scheme === 'always' || (scheme === 'first' && index === 0);
    if (prepend && !text.startsWith(rep)) text = rep + text;
    if (!split) { out.push({ text, special: false }); return; }
    let start = 0;
    for (let i = 1; i < text.length; i++) {
      if (text.startsWith(rep, i)) {
        if (i > start) out.push({ text: text.slice(start, i), special: false });
        start = i;
      }
    }
    if (text.length > start) out.push({ text: text.slice(start), special: false });
  });
  return out;
}

function whitespaceParts(parts) {
  const out = [];
  for (const part of parts) {
    if (part.special) { out.push(part); continue; }
    for (const piece of part.text.split(/\s+/u)) if (piece.length > 0) out.push({ text: piece, special: false });
  }
  return out;
}

// Min-heap of candidate merges keyed by (rank, left position). Each entry
// also keeps the two symbol strings it was made from, so an entry whose
// symbols have since changed is recognised as stale and dropped.
class MergeHeap {
  constructor() { this.rank = []; this.pos = []; this.a = []; this.b = []; }
  get size() { return this.rank.length; }
  less(i, j) { return this.rank[i] < this.rank[j] || (this.rank[i] === this.rank[j] && this.pos[i] < this.pos[j]); }
  swap(i, j) {
    for (const k of ['rank', 'pos', 'a', 'b']) { const t = this[k][i]; this[k][i] = this[k][j]; this[k][j] = t; }
  }
  push(rank, pos, a, b) {
    let i = this.rank.length;
    this.rank.push(rank); this.pos.push(pos); this.a.push(a); this.b.push(b);
    while (i > 0) {
      const p = (i - 1) >> 1;
      if (!this.less(i, p)) break;
      this.swap(i, p);
      i = p;
    }
  }
  // removes the top entry and returns [pos, a, b]
  pop() {
    const top = [this.pos[0], this.a[0], this.b[0]];
    const last = this.rank.length - 1;
    this.swap(0, last);
    this.rank.pop(); this.pos.pop(); this.a.pop(); this.b.pop();
    let i = 0;
    for (;;) {
      const l = 2 * i + 1, r = l + 1;
      let m = i;
      if (l < last && this.less(l, m)) m = l;
      if (r < last && this.less(r, m)) m = r;
      if (m === i) break;
      this.swap(i, m);
      i = m;
    }
    return top;
  }
}

class Gemma4Tokenizer {
  constructor(tokenizerJson, tokenizerConfig, generationConfig) {
    tokenizerConfig = tokenizerConfig || {};
    this.json = tokenizerJson;
    this.config = tokenizerConfig;
    this.generationConfig = generationConfig || {};
    this.model = tokenizerJson.model;
    if (!this.model || this.model.type !== 'BPE') {
      throw new Error(`Standalone tokenizer currently expects BPE tokenizer.json, got ${this.model ? this.model.type : undefined}.`);
    }
    this.vocab = new Map();
    this.idToToken = [];
    for (const token of Object.keys(this.model.vocab)) {
      const id = Number(this.model.vocab[token]);
      this.vocab.set(token, id);
      this.idToToken[id] = token;
    }
    // "left\0right" -> rank; a later duplicate of a pair replaces the earlier one
    this.mergeRanks = new Map();
    const merges = def(this.model.merges, []);
    for (let rank = 0; rank < merges.length; rank++) {
      const item = merges[rank];
      const pair = Array.isArray(item) ? item : String(item).split(' ');
      if (pair.length >= 2) this.mergeRanks.set(pair[0] + '\u0000' + pair[1], rank);
    }
    this.unkToken = def(this.model.unk_token, def(tokenizerConfig.unk_token, '<unk>'));
    this.unkId = Number(def(this.vocab.get(this.unkToken), 3));
    this.byteFallback = Boolean(this.model.byte_fallback);
    this.ignoreMerges = Boolean(this.model.ignore_merges);

    this.addedTokens = def(tokenizerJson.added_tokens, []).map((t) => Object.assign({}, t, { id: Number(t.id) }));
    this.addedById = new Map();
    for (const t of this.addedTokens) {
      this.idToToken[t.id] = t.content;
      this.vocab.set(t.content, t.id);
      this.addedById.set(t.id, t);
    }
    this.specialByText = new Map(this.addedTokens.filter((t) => t.special).map((t) => [t.content, t]));
    // Longest first: at one position the longest special text wins.
    this.specialTexts = Array.from(this.specialByText.keys()).sort((a, b) => b.length - a.length);
    this.specialRe = this.specialTexts.length
      ? new RegExp(this.specialTexts.map(escapeRegex).join('|'), 'g') : null;

    this.pretokenizers = flatten(tokenizerJson.pre_tokenizer, 'pretokenizers', 'pre_tokenizers');
    this.decoders = flatten(tokenizerJson.decoder, 'decoders');
    this.bosToken = def(tokenizerConfig.bos_token, '<bos>');
    this.eosToken = def(tokenizerConfig.eos_token, '<eos>');
    this.turnStartToken = def(tokenizerConfig.sot_token, '<|turn>');
    this.turnEndToken = def(tokenizerConfig.eot_token, '<turn|>');
    this.thinkToken = def(tokenizerConfig.think_token, '<|think|>');
  }

  // Reads tokenizer.json, tokenizer_config.json and, when present,
  // generation_config.json from a local directory (the reference fetches the
  // same three files from a base URL: standalone-tokenizer.js:372-403).
  static fromDirectorySync(dir) {
    const read = (name, required) => {
      const p = path.join(dir, name);
      if (!fs.existsSync(p)) {
        if (!required) return {};
        throw new Error(`Failed to load ${name}: no such file in ${dir}`);
      }
      return JSON.parse(fs.readFileSync(p, 'utf8'));
    };
    return new Gemma4Tokenizer(read('tokenizer.json', true), read('tokenizer_config.json', true),
      read('generation_config.json', false));
  }

  static async fromDirectory(dir) { return Gemma4Tokenizer.fromDirectorySync(dir); }

  // Special added tokens are cut out of the text first: the earliest match,
  // the longest at one position (standalone-tokenizer.js:405-448).
  splitAddedTokens(text) {
    if (!this.specialRe) return text.length ? [{ text, special: false }] : [];
    const out = [];
    let cursor = 0;
    this.specialRe.lastIndex = 0;
    let m;
    while ((m = this.specialRe.exec(text)) !== null) {
      if (m.index > cursor) out.push({ text: text.slice(cursor, m.index), special: false });
      out.push({ text: m[0], special: true });
      cursor = m.index + m[0].length;
    }
    if (cursor < text.length) out.push({ text: text.slice(cursor), special: false });
    return out;
  }

  pretokenize(text) {
    let parts = this.splitAddedTokens(normalize(text, this.json.normalizer));
    for (const cfg of this.pretokenizers) {
      if (cfg.type === 'Metaspace') parts = metaspaceParts(parts, cfg);
      else if (cfg.type === 'WhitespaceSplit') parts = whitespaceParts(parts);
      else if (cfg.type === 'Split') parts = splitParts(parts, cfg);
      else if (cfg.type === 'ByteLevel') throw new Error('ByteLevel pre-tokenizer is not expected for the Gemma 4 standalone path.');
      else throw new Error(`Unsupported pre-tokenizer: ${cfg.type}`);
    }
    return parts;
  }

  // Token ids of one pre-tokenized piece.
  encodePiece(piece) {
    if (this.ignoreMerges && this.vocab.has(piece)) return [this.vocab.get(piece)];
    const sym = [];
    for (const ch of piece) {
      if (this.vocab.has(ch) || !this.byteFallback) { sym.push(ch); continue; }
      for (const b of UTF8_ENCODER.encode(ch)) sym.push(byteToken(b));
    }
    const n = sym.length;
    // a lone symbol is looked up as it is, with no byte fallback (standalone-tokenizer.js:517-519)
    if (n < 2) return sym.map((s) => def(this.vocab.get(s), this.unkId));
    {
      const next = new Int32Array(n), prev = new Int32Array(n);
      for (let i = 0; i < n; i++) { next[i] = i + 1 < n ? i + 1 : -1; prev[i] = i - 1; }
      const heap = new MergeHeap();
      const offer = (l) => {
        const r = next[l];
        if (r < 0) return;
        const rank = this.mergeRanks.get(sym[l] + '\u0000' + sym[r]);
        if (rank !== undefined) heap.push(rank, l, sym[l], sym[r]);
      };
      for (let i = 0; i + 1 < n; i++) offer(i);
      while (heap.size) {
        const [l, a, b] = heap.pop();
        const r = next[l];
        if (sym[l] !== a || r < 0 || sym[r] !== b) continue;
        sym[l] = a + b;
        sym[r] = null;
        next[l] = next[r];
        if (next[r] >= 0) prev[next[r]] = l;
        if (prev[l] >= 0) offer(prev[l]);
        offer(l);
      }
    }
    const ids = [];
    for (const s of sym) {
      if (s === null) continue;
      const id = this.vocab.get(s);
      if (id !== undefined) { ids.push(id); continue; }
      if (this.byteFallback) {
        for (const b of UTF8_ENCODER.encode(s)) ids.push(def(this.vocab.get(byteToken(b)), this.unkId));
        continue;
      }
      ids.push(this.unkId);
    }
    return ids;
  }

  encode(text) {
    const ids = [];
    for (const part of this.pretokenize(text)) {
      if (part.special) {
        const t = this.specialByText.get(part.text);
        if (!t) throw new Error(`Special token not found: ${part.text}`);
        ids.push(t.id);
      } else if (part.text.length > 0) {
        for (const id of this.encodePiece(part.text)) ids.push(id);
      }
    }
    return ids;
  }

  // The decoder chain over token strings (standalone-tokenizer.js:600-704).
  // ByteFallback turns each run of <0xHH> tokens into text with a
  // non-fatal UTF-8 decode, so an invalid sequence becomes U+FFFD.
  decodeTokens(tokens) {
    let parts = tokens.slice();
    for (const d of this.decoders) {
      if (d.type === 'Replace') {
        const p = def(d.pattern, {});
        const from = def(p.String, p.Regex);
        const to = def(d.content, '');
        if (typeof from === 'string') parts = parts.map((t) => replaceEvery(t, from, to));
      } else if (d.type === 'ByteFallback') {
        const out = [];
        let bytes = [];
        const flush = () => {
          if (bytes.length) { out.push(UTF8_DECODER.decode(new Uint8Array(bytes))); bytes = []; }
        };
        for (const t of parts) {
          const v = parseByteToken(t);
          if (v === null) { flush(); out.push(t); } else bytes.push(v);
        }
        flush();
        parts = out;
      } else if (d.type === 'Fuse') {
        parts = [parts.join('')];
      } else if (d.type === 'Strip') {
        const content = def(d.content, ' ');
        const left = Number(def(d.start, def(d.left, 0)));
        const right = Number(def(d.stop, def(d.right, 0)));
        let v = parts.join('');
        for (let i = 0; i < left; i++) if (v.startsWith(content)) v = v.slice(content.length);
        for (let i = 0; i < right; i++) if (v.endsWith(content)) v = v.slice(0, -content.length);
        parts = [v];
      } else if (d.type === 'Metaspace') {
        let v = replaceEvery(parts.join(''), def(d.replacement, '▁'), ' ');
        if (def(d.prepend_scheme, 'always') !== 'never' && v.startsWith(' ')) v = v.slice(1);
        parts = [v];
      } else {
        throw new Error(`Unsupported decoder: ${d.type}`);
      }
    }
    return parts.join('');
  }

  // Unknown ids decode as the unknown-token text; special added tokens are
  // dropped unless skipSpecialTokens is false (standalone-tokenizer.js:706-734).
  decode(ids, opts) {
    const skip = opts && opts.skipSpecialTokens !== undefined ? opts.skipSpecialTokens : true;
    const tokens = [];
    for (const raw of ids) {
      const id = Number(raw);
      const token = this.idToToken[id];
      if (token === undefined || token === null) { tokens.push(this.unkToken); continue; }
      const added = this.addedById.get(id);
      if (skip && added && added.special) continue;
      tokens.push(token);
    }
    return this.decodeTokens(tokens);
  }

  // The user/assistant text-chat rendering of Gemma 4's template
  // (standalone-tokenizer.js:736-768): <bos>, an optional system turn that
  // enables thinking, one turn per message, then the open model turn.
  renderChat(messages, opts) {
    opts = opts || {};
    const addGenerationPrompt = opts.addGenerationPrompt !== undefined ? opts.addGenerationPrompt : true;
    let out = this.bosToken;
    if (opts.enableThinking) {
      out += this.turnStartToken + 'system\n' + this.thinkToken + '\n' + this.turnEndToken + '\n';
    }
    for (const m of messages) {
      if (m.role !== 'user' && m.role !== 'assistant') {
        throw new Error(`Standalone Gemma 4 text template currently supports user/assistant messages, got ${m.role}.`);
      }
      out += this.turnStartToken + m.role + '\n' + String(m.content) + this.turnEndToken + '\n';
    }
    if (addGenerationPrompt) out += this.turnStartToken + 'model\n';
    return out;
  }

  encodeChat(messages, opts) {
    const rendered = this.renderChat(messages, opts);
    return { rendered, ids: this.encode(rendered) };
  }

  // generation_config's eos_token_id (a number or a list) plus the ids of the
  // eos and end-of-turn tokens (standalone-tokenizer.js:782-814).
  stopTokenIds() {
    const out = new Set();
    const add = (v) => {
      if (v === undefined || v === null) return;
      if (Array.isArray(v)) { v.forEach(add); return; }
      out.add(Number(v));
    };
    add(this.generationConfig.eos_token_id);
    for (const t of [this.eosToken, this.turnEndToken]) {
      const id = this.vocab.get(t);
      if (id !== undefined) out.add(id);
    }
    return out;
  }

  describe() {
    return {
      modelType: this.model.type,
      vocabSize: this.vocab.size,
      merges: this.mergeRanks.size,
      byteFallback: this.byteFallback,
      pretokenizers: this.pretokenizers.map((p) => p.type),
      decoders: this.decoders.map((d) => d.type),
      specialTokens: this.specialByText.size,
    };
  }
}

module.exports = { Gemma4Tokenizer, byteToken, parseByteToken };
