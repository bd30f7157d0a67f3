// Token-prefix SHA-256 hashes for the reuse gate and the KV store (host code).
//
// Reference semantics (src/chunkkv/store/keys.py:15-20):
//   h = sha256(); h.update(len(tokens).to_bytes(4, "little"))
//   for t in tokens: h.update(t.to_bytes(4, "little"))
//   return h.hexdigest()
// called as token_hash(req.tokens[:seg.start]) once per segment by the gate
// (src/chunkkv/gate/gate.py:42) and again for every stored segment (src/chunkkv/runtime.py:89):
// one Python update per token, O(N x segments) per request.
//
// Here every prefix's message (4-byte length, then 4-byte tokens, little-endian) is hashed
// straight out of one converted copy of the request's tokens: the length header differs between
// prefixes, so no hash state is shared, and prefixes are independent work items spread over
// threads, longest first. SHA-256 follows FIPS 180-4; on x86 CPUs with the SHA extensions the
// compression function runs on them (sha256rnds2 / sha256msg1 / sha256msg2), chosen at run time.
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <thread>
#include <vector>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

#include "chunkkv_amd.h"

namespace {

// FIPS 180-4 section 4.2.2: first 32 bits of the fractional parts of the cube roots of the
// first 64 primes; section 5.3.3: of the square roots of the first 8 primes.
const uint32_t kK[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
const uint32_t kH0[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                         0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
inline uint32_t load_be32(const uint8_t* p) {
  return ((uint32_t)p[0] << 24) | ((uint32_t)p[1] << 16) | ((uint32_t)p[2] << 8) | (uint32_t)p[3];
}

// FIPS 180-4 section 6.2.2, one 64-byte block at a time.
void compress_portable(uint32_t st[8], const uint8_t* data, size_t n_blocks) {
  for (size_t b = 0; b < n_blocks; ++b, data += 64) {
    uint32_t w[64];
    for (int i = 0; i < 16; ++i) w[i] = load_be32(data + 4 * i);
    for (int i = 16; i < 64; ++i) {
      const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
      const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
      w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = st[0], bb = st[1], c = st[2], d = st[3], e = st[4], f = st[5], g = st[6], h = st[7];
    for (int i = 0; i < 64; ++i) {
      const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + kK[i] + w[i];
      const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & bb) ^ (a & c) ^ (bb & c));
      h = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = bb;
      bb = a;
      a = t1 + t2;
    }
    st[0] += a;
    st[1] += bb;
    st[2] += c;
    st[3] += d;
    st[4] += e;
    st[5] += f;
    st[6] += g;
    st[7] += h;
  }
}

#if defined(__x86_64__)
// The same compression on the x86 SHA extensions. The instructions keep the working state as
// two registers, (A, B, E, F) and (C, D, G, H) in lanes 3..0, advance it two rounds per
// sha256rnds2 with the round's W + K in the low lanes of the message operand, and extend the
// message schedule four words at a time (sha256msg1 / sha256msg2 with the alignr term).
__attribute__((target("sha,sse4.1,ssse3"))) void compress_shani(uint32_t st[8], const uint8_t* data,
                                                                size_t n_blocks) {
  const __m128i bswap = _mm_set_epi64x(0x0c0d0e0f08090a0bLL, 0x0405060700010203LL);
  __m128i t = _mm_loadu_si128((const __m128i*)&st[0]);  // a b c d (lane 0 = a)
  __m128i s1 = _mm_loadu_si128((const __m128i*)&st[4]);  // e f g h
  t = _mm_shuffle_epi32(t, 0xB1);                         // b a d c
  s1 = _mm_shuffle_epi32(s1, 0x1B);                       // h g f e
  __m128i s0 = _mm_alignr_epi8(t, s1, 8);                 // f e b a: (A, B, E, F) in lanes 3..0
  s1 = _mm_blend_epi16(s1, t, 0xF0);                      // h g d c: (C, D, G, H) in lanes 3..0
  for (size_t b = 0; b < n_blocks; ++b, data += 64) {
    const __m128i s0_in = s0, s1_in = s1;
    __m128i m[4];
    for (int i = 0; i < 4; ++i) m[i] = _mm_shuffle_epi8(_mm_loadu_si128((const __m128i*)(data + 16 * i)), bswap);
    for (int g = 0; g < 16; ++g) {  // rounds 4g .. 4g + 3
      __m128i msg = _mm_add_epi32(m[g & 3], _mm_loadu_si128((const __m128i*)&kK[4 * g]));
      s1 = _mm_sha256rnds2_epu32(s1, s0, msg);
      if (g >= 3 && g <= 14) {  // W of rounds 4(g+1) .. 4(g+1) + 3
        const __m128i tmp = _mm_alignr_epi8(m[g & 3], m[(g + 3) & 3], 4);
        m[(g + 1) & 3] = _mm_sha256msg2_epu32(_mm_add_epi32(m[(g + 1) & 3], tmp), m[g & 3]);
      }
      msg = _mm_shuffle_epi32(msg, 0x0E);
      s0 = _mm_sha256rnds2_epu32(s0, s1, msg);
      if (g >= 1 && g <= 12) m[(g + 3) & 3] = _mm_sha256msg1_epu32(m[(g + 3) & 3], m[g & 3]);
    }
    s0 = _mm_add_epi32(s0, s0_in);
    s1 = _mm_add_epi32(s1, s1_in);
  }
  t = _mm_shuffle_epi32(s0, 0x1B);   // a b e f
  s1 = _mm_shuffle_epi32(s1, 0xB1);  // g h c d
  s0 = _mm_blend_epi16(t, s1, 0xF0);  // a b c d
  s1 = _mm_alignr_epi8(s1, t, 8);     // e f g h
  _mm_storeu_si128((__m128i*)&st[0], s0);
  _mm_storeu_si128((__m128i*)&st[4], s1);
}
#endif

typedef void (*CompressFn)(uint32_t*, const uint8_t*, size_t);

CompressFn pick_compress() {
  const char* force = std::getenv("CKV_SHA256_PORTABLE");
  if (force != nullptr && force[0] == '1') return &compress_portable;
#if defined(__x86_64__)
  __builtin_cpu_init();
  if (__builtin_cpu_supports("sha") && __builtin_cpu_supports("sse4.1")) return &compress_shani;
#endif
  return &compress_portable;
}

// SHA-256 of LE32(n) || tok[0 .. n) where `tok` holds the tokens as LE32 bytes.
void hash_prefix(const uint8_t* tok, uint32_t n, uint8_t out[32], CompressFn compress) {
  uint32_t st[8];
  memcpy(st, kH0, sizeof(st));
  const uint64_t body = 4ull * n;     // token bytes
  const uint64_t total = 4 + body;    // message bytes
  uint8_t blk[128];
  uint64_t done = 0;                   // token bytes already compressed
  bool header_done = false;
  if (total >= 64) {                   // first block: the length header and 60 token bytes
    blk[0] = (uint8_t)n;
    blk[1] = (uint8_t)(n >> 8);
    blk[2] = (uint8_t)(n >> 16);
    blk[3] = (uint8_t)(n >> 24);
    memcpy(blk + 4, tok, 60);
    compress(st, blk, 1);
    done = 60;
    header_done = true;
    const uint64_t full = (body - done) / 64;  // whole blocks straight from the token bytes
    if (full) compress(st, tok + done, (size_t)full);
    done += 64 * full;
  }
  size_t len = 0;  // the rest of the message, then the padding (section 5.1.1)
  if (!header_done) {
    blk[0] = (uint8_t)n;
    blk[1] = (uint8_t)(n >> 8);
    blk[2] = (uint8_t)(n >> 16);
    blk[3] = (uint8_t)(n >> 24);
    len = 4;
  }
  memcpy(blk + len, tok + done, (size_t)(body - done));
  len += (size_t)(body - done);
  blk[len++] = 0x80;
  const size_t end = len <= 56 ? 64 : 128;
  memset(blk + len, 0, end - 8 - len);
  const uint64_t bits = total * 8;
  for (int i = 0; i < 8; ++i) blk[end - 1 - i] = (uint8_t)(bits >> (8 * i));
  compress(st, blk, end / 64);
  for (int i = 0; i < 8; ++i) {
    out[4 * i] = (uint8_t)(st[i] >> 24);
    out[4 * i + 1] = (uint8_t)(st[i] >> 16);
    out[4 * i + 2] = (uint8_t)(st[i] >> 8);
    out[4 * i + 3] = (uint8_t)st[i];
  }
}

}  // namespace

extern "C" int32_t ckv_token_hash_prefixes(const int64_t* tokens, int64_t n_tokens, const int64_t* starts,
                                           int32_t n_starts, uint8_t* digests, int32_t n_threads) {
  if (n_tokens < 0 || n_starts < 0 || (n_starts > 0 && (starts == nullptr || digests == nullptr)) ||
      (n_tokens > 0 && tokens == nullptr))
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_tokens > 0xffffffffLL) return CKV_ERR_TOO_LARGE;  // the length header is 4 bytes
  int64_t longest = 0;
  for (int32_t i = 0; i < n_starts; ++i) {
    if (starts[i] < 0 || starts[i] > n_tokens) return CKV_ERR_OUT_OF_RANGE;
    longest = std::max(longest, starts[i]);
  }
  // the tokens of the longest prefix as little-endian 4-byte words; an id outside [0, 2^32)
  // cannot be encoded (the reference's int.to_bytes raises OverflowError)
  std::vector<uint8_t> buf((size_t)longest * 4 + 64);
  for (int64_t i = 0; i < longest; ++i) {
    const int64_t t = tokens[i];
    if (t < 0 || t > 0xffffffffLL) return CKV_ERR_OUT_OF_RANGE;
    const uint32_t u = (uint32_t)t;
    memcpy(&buf[(size_t)i * 4], &u, 4);  // x86 and the GPU hosts are little-endian
  }
  const CompressFn compress = pick_compress();
  std::vector<int32_t> order((size_t)n_starts);
  for (int32_t i = 0; i < n_starts; ++i) order[(size_t)i] = i;
  std::sort(order.begin(), order.end(), [&](int32_t a, int32_t b) { return starts[a] > starts[b]; });
  int workers = n_threads > 0 ? n_threads : (int)std::thread::hardware_concurrency();
  int64_t work = 0;
  for (int32_t i = 0; i < n_starts; ++i) work += starts[i] + 16;
  workers = std::max(1, std::min({workers, 16, n_starts, (int)(work / 8192) + 1}));  // ~32 KB of message each
  std::atomic<int32_t> next{0};
  auto run = [&]() {
    for (int32_t k; (k = next.fetch_add(1)) < n_starts;) {
      const int32_t i = order[(size_t)k];
      hash_prefix(buf.data(), (uint32_t)starts[i], digests + 32 * (size_t)i, compress);
    }
  };
  std::vector<std::thread> pool;
  for (int w = 1; w < workers; ++w) pool.emplace_back(run);
  run();
  for (auto& th : pool) th.join();
  return CKV_OK;
}
