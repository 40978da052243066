// tq_entropy.hip -- host-side Huffman bit packing for entropy-coded code storage
// (the byte format of turboquant_kv/entropy.py:162-231).
//
// Stream: uint32 LE n_symbols, uint32 LE n_bits, then the symbols' code words
// concatenated most significant bit first, the last byte zero-padded.  The code table is
// built by the caller (the Huffman tree is a few dozen nodes); these functions do the
// per-symbol work: the reference builds a '0'/'1' Python string per symbol and parses it
// back character by character.

#include "tq_common.h"

#include <algorithm>
#include <unordered_map>
#include <vector>

using namespace tq;

extern "C" {

int tq_huffman_encode(const uint8_t* codes, int64_t n, const uint64_t* code_words,
                      const uint8_t* code_lens, int32_t n_levels, uint8_t* out, size_t out_capacity,
                      size_t* out_bytes) {
  TQ_REQUIRE(n >= 0 && n <= 0xFFFFFFFFll, "symbol count must fit in 32 bits");
  TQ_REQUIRE(n_levels >= 1 && n_levels <= 256, "n_levels must be in [1, 256]");
  TQ_REQUIRE(code_words && code_lens && out && out_bytes && (n == 0 || codes), "null pointer argument");
  for (int s = 0; s < n_levels; ++s)
    TQ_REQUIRE(code_lens[s] >= 1 && code_lens[s] <= 64, "code length of symbol %d out of range", s);
  uint64_t nbits = 0;
  for (int64_t i = 0; i < n; ++i) {
    TQ_REQUIRE(codes[i] < n_levels, "symbol %d at %lld out of range", (int)codes[i], (long long)i);
    nbits += code_lens[codes[i]];
  }
  TQ_REQUIRE(nbits <= 0xFFFFFFFFull, "bit count must fit in 32 bits");
  const size_t need = 8 + (size_t)((nbits + 7) / 8);
  *out_bytes = need;
  TQ_REQUIRE(out_capacity >= need, "output too small: need %zu bytes", need);
  const uint32_t h[2] = {(uint32_t)n, (uint32_t)nbits};
  for (int k = 0; k < 2; ++k)
    for (int b = 0; b < 4; ++b) out[4 * k + b] = (uint8_t)(h[k] >> (8 * b));
  uint8_t* body = out + 8;
  std::fill(body, body + (need - 8), (uint8_t)0);
  // Bits accumulate MSB first in a 64-bit register and leave it a byte at a time.
  uint64_t acc = 0;
  int held = 0;
  size_t pos = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int len = code_lens[codes[i]];
    uint64_t w = code_words[codes[i]];
    int left = len;
    while (left > 0) {
      const int take = left < 56 - held ? left : 56 - held;
      const uint64_t part = (w >> (left - take)) & ((take == 64) ? ~0ull : ((1ull << take) - 1));
      acc = (acc << take) | part;
      held += take;
      left -= take;
      while (held >= 8) {
        body[pos++] = (uint8_t)(acc >> (held - 8));
        held -= 8;
      }
    }
  }
  if (held > 0) body[pos++] = (uint8_t)(acc << (8 - held));
  return TQ_OK;
}

int tq_huffman_decode(const uint8_t* data, size_t data_bytes, int64_t n_symbols,
                      const uint64_t* code_words, const uint8_t* code_lens, const int32_t* symbols,
                      int32_t n_codes, uint8_t* out, int64_t* n_out) {
  TQ_REQUIRE(data && data_bytes >= 8 && n_out, "null pointer or short stream");
  TQ_REQUIRE(n_codes >= 1 && code_words && code_lens && symbols, "empty code table");
  uint32_t stored_n = 0, stored_bits = 0;
  for (int b = 0; b < 4; ++b) {
    stored_n |= (uint32_t)data[b] << (8 * b);
    stored_bits |= (uint32_t)data[4 + b] << (8 * b);
  }
  if (n_symbols < 0) n_symbols = stored_n;
  TQ_REQUIRE(n_symbols == 0 || out, "null pointer argument");
  const uint64_t avail = (uint64_t)(data_bytes - 8) * 8;
  const uint64_t nbits = stored_bits < avail ? stored_bits : avail;
  // (length, word) -> symbol; a later table entry for the same code word replaces an
  // earlier one, as a dict built from the table in order does
  std::unordered_map<uint64_t, int32_t> table;
  int maxlen = 0;
  for (int c = 0; c < n_codes; ++c) {
    TQ_REQUIRE(code_lens[c] >= 1 && code_lens[c] <= 56, "code length out of range");
    table[((uint64_t)code_lens[c] << 56) | code_words[c]] = symbols[c];
    if (code_lens[c] > maxlen) maxlen = code_lens[c];
  }
  const uint8_t* body = data + 8;
  const size_t body_bytes = data_bytes - 8;
  int64_t done = 0;
  if (maxlen <= 20) {
    // Window table: entry w of the 2^maxlen windows holds the shortest code word that
    // prefixes w ((length << 16) | symbol; 0: none) -- the word the bit-by-bit walk below
    // would match first.  A word longer than the bits left, or no word at all, ends the
    // stream as the walk does.
    std::vector<uint32_t> peek((size_t)1 << maxlen, 0u);
    for (const auto& kv : table) {
      const int l = (int)(kv.first >> 56);
      const uint64_t word = kv.first & ((1ull << 56) - 1);
      if (word >> l) continue;  // wider than its length: never matched
      const uint32_t e = ((uint32_t)l << 16) | (uint32_t)(kv.second & 0xFFFF);
      const size_t base = (size_t)word << (maxlen - l), span = (size_t)1 << (maxlen - l);
      for (size_t i = base; i < base + span; ++i)
        if (peek[i] == 0 || (int)(peek[i] >> 16) > l) peek[i] = e;
    }
    const uint32_t wmask = (1u << maxlen) - 1;
    uint64_t p = 0;
    while (done < n_symbols && p < nbits) {
      const size_t at = (size_t)(p >> 3);
      uint64_t v = 0;  // 32 bits from byte `at`, zeros past the body
      for (int i = 0; i < 4; ++i) v = (v << 8) | (at + i < body_bytes ? body[at + i] : 0u);
      const uint32_t e = peek[(uint32_t)(v >> (32 - (int)(p & 7) - maxlen)) & wmask];
      if (e == 0 || p + (e >> 16) > nbits) break;
      out[done++] = (uint8_t)(e & 0xFFFF);
      p += e >> 16;
    }
    *n_out = done;
    return TQ_OK;
  }
  uint64_t cur = 0;
  int len = 0;
  for (uint64_t p = 0; p < nbits && done < n_symbols; ++p) {
    cur = (cur << 1) | ((body[p >> 3] >> (7 - (p & 7))) & 1u);
    ++len;
    const auto it = table.find(((uint64_t)len << 56) | cur);
    if (it != table.end()) {
      out[done++] = (uint8_t)it->second;
      cur = 0;
      len = 0;
    } else if (len >= maxlen) {
      // no code word this long: the reference keeps extending its prefix forever and
      // decodes nothing further
      break;
    }
  }
  *n_out = done;
  return TQ_OK;
}

}  // extern "C"
