// ztcp_keyring.cpp -- session key ring of the cold-page codec (host code).
//
// Native counterpart of EphemeralSessionKeyRing
// (research/baseline_codec/fused_quant_crypto.py, "fqc", lines 99-659); the
// C ABI is declared in include/ztcp_keyring.h.  Each method keeps the
// reference's checks, their order, its error kinds and messages, and its
// state transitions:
//   * keys: HMAC-SHA256 derivation per (tenant, session, generation) from the
//     deployment pepper and 32 fresh random bytes (fqc:196-239);
//   * nonce burn: every 96-bit ChaCha20 nonce of an egress batch is checked
//     and burned before any encryption (fqc:257-341);
//   * freshness: per-slot watermarks (model, layer, head group, token hash)
//     only move forward (fqc:397-434, fqc:473-603);
//   * crypto-shred: key buffers and in-flight reservation copies are zeroed,
//     in-flight reservations revoked, the generation retired (fqc:620-658).
#include <sys/random.h>

#include <array>
#include <cerrno>
#include <cinttypes>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include "../../include/ztcp_keyring.h"

// ---------------------------------------------------------------------------
// SHA-256 (FIPS 180-4 section 6.2) and HMAC (RFC 2104).
// ---------------------------------------------------------------------------
namespace {

constexpr uint32_t kSha256K[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
    0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
    0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
    0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
    0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
    0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

struct Sha256 {
    uint32_t h[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                     0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    uint8_t buf[64];
    size_t fill = 0;
    uint64_t total = 0;

    void block(const uint8_t* p) {
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], k = h[7];
        for (int i = 0; i < 64; ++i) {
            const uint32_t t1 = k + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + kSha256K[i] + w[i];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            k = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += k;
    }
    void update(const uint8_t* p, size_t n) {
        total += n;
        while (n) {
            const size_t take = std::min(n, (size_t)64 - fill);
            std::memcpy(buf + fill, p, take);
            fill += take; p += take; n -= take;
            if (fill == 64) { block(buf); fill = 0; }
        }
    }
    void final(uint8_t out[32]) {
        const uint64_t bits = total * 8u;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (fill != 56) update(&zero, 1);
        uint8_t len[8];
        for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
        update(len, 8);
        for (int i = 0; i < 8; ++i) {
            out[4 * i] = (uint8_t)(h[i] >> 24); out[4 * i + 1] = (uint8_t)(h[i] >> 16);
            out[4 * i + 2] = (uint8_t)(h[i] >> 8); out[4 * i + 3] = (uint8_t)h[i];
        }
        volatile uint8_t* v = buf;  // the block buffer may hold key material
        for (int i = 0; i < 64; ++i) v[i] = 0;
    }
};

void hmac_sha256(const uint8_t* key, size_t key_len, const uint8_t* a, size_t na, const uint8_t* b, size_t nb,
                 uint8_t out[32]) {
    uint8_t k[64] = {0}, pad[64];
    if (key_len > 64) {
        Sha256 s;
        s.update(key, key_len);
        s.final(k);
    } else {
        std::memcpy(k, key, key_len);
    }
    for (int i = 0; i < 64; ++i) pad[i] = k[i] ^ 0x36;
    uint8_t inner[32];
    Sha256 si;
    si.update(pad, 64);
    si.update(a, na);
    if (nb) si.update(b, nb);
    si.final(inner);
    for (int i = 0; i < 64; ++i) pad[i] = k[i] ^ 0x5c;
    Sha256 so;
    so.update(pad, 64);
    so.update(inner, 32);
    so.final(out);
    volatile uint8_t* vk = k;
    volatile uint8_t* vp = pad;
    volatile uint8_t* vi = inner;
    for (int i = 0; i < 64; ++i) { vk[i] = 0; vp[i] = 0; }
    for (int i = 0; i < 32; ++i) vi[i] = 0;
}

// ---------------------------------------------------------------------------
// Key ring state.
// ---------------------------------------------------------------------------

using Key = std::pair<std::string, std::string>;  // (tenant_id, session_id)
using Buf = std::array<uint8_t, 32>;

void wipe(Buf& b) {
    volatile uint8_t* v = b.data();
    for (size_t i = 0; i < b.size(); ++i) v[i] = 0;
}
bool nonzero(const Buf& b) {
    uint8_t acc = 0;
    for (uint8_t x : b) acc |= x;
    return acc != 0;
}

// 96-bit ChaCha20 nonce: sequence (8 bytes LE) || (layer << 16 | head group) (4 bytes LE) (fqc:157-166).
struct Nonce {
    uint64_t seq;
    uint32_t loc;
    bool operator==(const Nonce& o) const { return seq == o.seq && loc == o.loc; }
};
struct NonceHash {
    size_t operator()(const Nonce& n) const {
        return std::hash<uint64_t>()(n.seq * 0x9E3779B97F4A7C15ull ^ n.loc);
    }
};

// Logical KV page slot (model hash, layer, head group, token hash).
struct Slot {
    uint32_t model;
    uint16_t layer, head_group;
    uint64_t token;
    bool operator==(const Slot& o) const {
        return model == o.model && layer == o.layer && head_group == o.head_group && token == o.token;
    }
};
struct SlotHash {
    size_t operator()(const Slot& s) const {
        return std::hash<uint64_t>()(s.token * 0x9E3779B97F4A7C15ull ^ ((uint64_t)s.model << 32) ^
                                     ((uint64_t)s.layer << 16) ^ s.head_group);
    }
};

std::string hex(const Nonce& n) {
    uint8_t b[12];
    for (int i = 0; i < 8; ++i) b[i] = (uint8_t)(n.seq >> (8 * i));
    for (int i = 0; i < 4; ++i) b[8 + i] = (uint8_t)(n.loc >> (8 * i));
    static const char* d = "0123456789abcdef";
    std::string s;
    for (uint8_t x : b) { s += d[x >> 4]; s += d[x & 15]; }
    return s;
}

std::string key_repr(const Key& k) { return "('" + k.first + "', '" + k.second + "')"; }

thread_local std::string t_last_error;

struct Error {
    int code;
    std::string msg;
};

}  // namespace

struct ztcp_reservation {
    uint64_t generation = 0;
    Buf enc{}, mac{};
    bool revoked = false;
    std::vector<std::pair<Slot, uint64_t>> slots;  // staged slot watermarks to commit
    uint64_t last_seq = 0;
    Key key;

    void zeroize() { wipe(enc); wipe(mac); }
};

struct ztcp_keyring {
    std::vector<uint8_t> pepper;
    std::mutex mu;
    std::map<Key, std::pair<Buf, Buf>> active;              // _active_keys / _active_key_buffers
    std::map<Key, uint64_t> session_gen;                    // _session_generations
    std::map<Key, uint64_t> shredded_gen;                   // _shredded_generations
    std::map<Key, std::unordered_set<Nonce, NonceHash>> used_nonces;
    std::map<Key, std::unordered_map<Slot, uint64_t, SlotHash>> slot_latest;
    std::map<Key, uint64_t> session_max;
    std::map<std::pair<Key, uint64_t>, std::vector<ztcp_reservation*>> inflight;

    uint64_t get(const std::map<Key, uint64_t>& m, const Key& k, uint64_t dflt = 0) const {
        auto it = m.find(k);
        return it == m.end() ? dflt : it->second;
    }

    // _ensure_active_generation_locked (fqc:168-194)
    uint64_t ensure_active(const Key& k) {
        auto it = active.find(k);
        if (it == active.end()) throw Error{ZTCP_KR_ESHREDDED, "Session " + key_repr(k) + " key is missing or crypto-shredded"};
        if (!nonzero(it->second.first) || !nonzero(it->second.second))
            throw Error{ZTCP_KR_ESHREDDED, "Session " + key_repr(k) + " key buffer was zeroized or crypto-shredded"};
        auto g = session_gen.find(k);
        if (g == session_gen.end()) g = session_gen.emplace(k, get(shredded_gen, k) + 1).first;
        return g->second;
    }

    // derive_or_get (fqc:196-239); `secret` = the 32 random bytes
    void derive(const Key& k, const uint8_t* secret) {
        const uint64_t gen = std::max(get(session_gen, k), get(shredded_gen, k)) + 1;
        session_gen[k] = gen;
        const std::string label = k.first + ":" + k.second + ":gen=" + std::to_string(gen) + ":";
        uint8_t prk[32];
        hmac_sha256(pepper.data(), pepper.size(), (const uint8_t*)label.data(), label.size(), secret, 32, prk);
        Buf enc, mac;
        static const char enc_info[] = "ztcp-cold-page-enc-v1\x01";
        static const char mac_info[] = "ztcp-cold-page-mac-v1\x02";
        hmac_sha256(prk, 32, (const uint8_t*)enc_info, sizeof(enc_info) - 1, nullptr, 0, enc.data());
        hmac_sha256(prk, 32, (const uint8_t*)mac_info, sizeof(mac_info) - 1, nullptr, 0, mac.data());
        volatile uint8_t* vp = prk;
        for (int i = 0; i < 32; ++i) vp[i] = 0;
        active[k] = {enc, mac};
        wipe(enc);
        wipe(mac);
        used_nonces[k].clear();
        slot_latest[k].clear();
        session_max[k] = 0;
        inflight[{k, gen}];
    }

    void derive_random(const Key& k) {
        uint8_t secret[32];
        size_t got = 0;
        while (got < sizeof(secret)) {
            const ssize_t r = getrandom(secret + got, sizeof(secret) - got, 0);
            if (r < 0) {
                if (errno == EINTR) continue;
                throw Error{ZTCP_KR_ERANDOM, "os random source failed"};
            }
            got += (size_t)r;
        }
        derive(k, secret);
        volatile uint8_t* v = secret;
        for (int i = 0; i < 32; ++i) v[i] = 0;
    }

    void ensure_derived(const Key& k) {
        if (active.find(k) == active.end()) derive_random(k);
    }

    // _resolve_reservation_generation_locked + the revocation test shared by
    // begin_egress_execution and commit_egress (fqc:356-434)
    void check_reservation(const Key& k, ztcp_reservation* r, const char* when) {
        const uint64_t g = r->generation;
        if (r->revoked || active.find(k) == active.end() || get(session_gen, k) != g || get(shredded_gen, k) >= g) {
            r->zeroize();
            throw Error{ZTCP_KR_ESHREDDED, "Session (" + k.first + ", " + k.second + ") generation " +
                                               std::to_string(g) + " was crypto-shredded " + when};
        }
    }

    // _zeroize_and_remove_session (fqc:620-645)
    bool shred(const Key& k) {
        const uint64_t gen = get(session_gen, k, 1);
        auto it = active.find(k);
        const bool existed = it != active.end();
        if (existed) {
            wipe(it->second.first);
            wipe(it->second.second);
            active.erase(it);
        }
        auto inf = inflight.find({k, gen});
        if (inf != inflight.end()) {
            for (ztcp_reservation* r : inf->second) {
                r->revoked = true;
                r->zeroize();
            }
            inflight.erase(inf);
        }
        used_nonces.erase(k);
        slot_latest.erase(k);
        session_max.erase(k);
        if (existed) shredded_gen[k] = std::max(get(shredded_gen, k), gen);
        return existed;
    }

    void unlink(ztcp_reservation* r) {
        auto inf = inflight.find({r->key, r->generation});
        if (inf == inflight.end()) return;
        auto& v = inf->second;
        for (size_t i = 0; i < v.size(); ++i)
            if (v[i] == r) { v.erase(v.begin() + (long)i); break; }
    }
};

namespace {

template <class F>
int guarded(ztcp_keyring* kr, F&& f) {
    t_last_error.clear();
    if (!kr) {
        t_last_error = "key ring is NULL";
        return ZTCP_KR_EINVAL;
    }
    try {
        std::lock_guard<std::mutex> lock(kr->mu);
        return f();
    } catch (const Error& e) {
        t_last_error = e.msg;
        return e.code;
    } catch (const std::bad_alloc&) {
        t_last_error = "out of memory";
        return ZTCP_KR_ENOMEM;
    }
}

bool strings_ok(const char* a, const char* b) { return a && b; }

void copy_out(const Buf& b, uint8_t* out) {
    if (out) std::memcpy(out, b.data(), 32);
}

int check_stale(uint64_t seq, uint64_t prev) {
    if (seq < prev)
        throw Error{ZTCP_KR_ESTALE, "STALE_PAGE_REPLAY: Cannot encode cold page with stale sequence_nonce=" +
                                        std::to_string(seq) + " < latest=" + std::to_string(prev)};
    return 0;
}

}  // namespace

extern "C" {

int ztcp_keyring_create(const uint8_t* pepper, size_t pepper_len, ztcp_keyring** out) {
    t_last_error.clear();
    if (!out || (!pepper && pepper_len)) {
        t_last_error = "invalid argument";
        return ZTCP_KR_EINVAL;
    }
    if (pepper_len < 32) {  // fqc:155-157
        t_last_error = "deployment_pepper must be at least 32 bytes";
        return ZTCP_KR_EINVAL;
    }
    try {
        ztcp_keyring* kr = new ztcp_keyring;
        kr->pepper.assign(pepper, pepper + pepper_len);
        *out = kr;
        return 0;
    } catch (const std::bad_alloc&) {
        t_last_error = "out of memory";
        return ZTCP_KR_ENOMEM;
    }
}

void ztcp_keyring_destroy(ztcp_keyring* kr) {
    if (!kr) return;
    {
        std::lock_guard<std::mutex> lock(kr->mu);
        for (auto& kv : kr->active) {
            wipe(kv.second.first);
            wipe(kv.second.second);
        }
        for (auto& kv : kr->inflight)
            for (ztcp_reservation* r : kv.second) {
                r->revoked = true;
                r->zeroize();
                delete r;
            }
        kr->inflight.clear();
        volatile uint8_t* v = kr->pepper.data();
        for (size_t i = 0; i < kr->pepper.size(); ++i) v[i] = 0;
    }
    delete kr;
}

int ztcp_keyring_derive_or_get(ztcp_keyring* kr, const char* tenant, const char* session, uint8_t enc_key[32],
                               uint8_t mac_key[32], uint64_t* generation) {
    return guarded(kr, [&] {
        if (!strings_ok(tenant, session)) throw Error{ZTCP_KR_EINVAL, "tenant and session ids are required"};
        const Key k{tenant, session};
        uint64_t gen;
        if (kr->active.count(k)) {
            gen = kr->ensure_active(k);
        } else {
            kr->derive_random(k);
            gen = kr->get(kr->session_gen, k);
        }
        const auto& kb = kr->active.at(k);
        copy_out(kb.first, enc_key);
        copy_out(kb.second, mac_key);
        if (generation) *generation = gen;
        return 0;
    });
}

int ztcp_keyring_derive_with_secret_for_test(ztcp_keyring* kr, const char* tenant, const char* session,
                                             const uint8_t secret[32], uint8_t enc_key[32], uint8_t mac_key[32],
                                             uint64_t* generation) {
    return guarded(kr, [&] {
        if (!strings_ok(tenant, session) || !secret) throw Error{ZTCP_KR_EINVAL, "invalid argument"};
        const Key k{tenant, session};
        if (kr->active.count(k)) throw Error{ZTCP_KR_EINVAL, "session already has keys"};
        kr->derive(k, secret);
        const auto& kb = kr->active.at(k);
        copy_out(kb.first, enc_key);
        copy_out(kb.second, mac_key);
        if (generation) *generation = kr->get(kr->session_gen, k);
        return 0;
    });
}

int ztcp_keyring_next_sequence_nonce(ztcp_keyring* kr, const char* tenant, const char* session, uint64_t count,
                                     uint64_t* base) {
    return guarded(kr, [&] {
        if (!strings_ok(tenant, session) || !base) throw Error{ZTCP_KR_EINVAL, "invalid argument"};
        if (count < 1) throw Error{ZTCP_KR_EINVAL, "count must be >= 1"};
        const Key k{tenant, session};
        kr->ensure_derived(k);
        kr->ensure_active(k);
        const uint64_t b = kr->get(kr->session_max, k) + 1;
        kr->session_max[k] = b + count - 1;
        *base = b;
        return 0;
    });
}

int ztcp_keyring_preflight_egress(ztcp_keyring* kr, const char* tenant, const char* session, uint32_t model_id_hash,
                                  uint16_t layer_id, uint16_t head_group_id, uint64_t base_sequence_nonce,
                                  const uint64_t* token_hashes, size_t n, ztcp_reservation** out) {
    return guarded(kr, [&] {
        if (!strings_ok(tenant, session) || !out || (!token_hashes && n)) throw Error{ZTCP_KR_EINVAL, "invalid argument"};
        if (n == 0) throw Error{ZTCP_KR_EINVAL, "token_hashes must be non-empty"};
        const Key k{tenant, session};
        kr->ensure_derived(k);
        const uint64_t gen = kr->ensure_active(k);
        auto& used = kr->used_nonces[k];
        auto& marks = kr->slot_latest[k];
        const uint32_t loc = ((uint32_t)layer_id << 16) | head_group_id;
        std::unordered_set<Nonce, NonceHash> staged;
        std::unordered_map<Slot, uint64_t, SlotHash> staged_slots;
        staged.reserve(n * 2);
        staged_slots.reserve(n * 2);
        for (size_t i = 0; i < n; ++i) {
            const uint64_t seq = base_sequence_nonce + i;  // wraps mod 2^64 as the reference masks it
            const Slot s{model_id_hash, layer_id, head_group_id, token_hashes[i]};
            auto st = staged_slots.find(s);
            uint64_t prev = 0;
            if (st != staged_slots.end()) {
                prev = st->second;
            } else {
                auto m = marks.find(s);
                if (m != marks.end()) prev = m->second;
            }
            check_stale(seq, prev);
            const Nonce nn{seq, loc};
            if (used.count(nn) || staged.count(nn))
                throw Error{ZTCP_KR_ENONCE, "NONCE_REUSE_DETECTED: Final 96-bit ChaCha20 nonce " + hex(nn) +
                                                " already used under session " + key_repr(k)};
            staged.insert(nn);
            staged_slots[s] = seq;
        }
        // all checks passed: register the key-bearing reservation and burn the nonces
        ztcp_reservation* r = new ztcp_reservation;
        const auto& kb = kr->active.at(k);
        r->generation = gen;
        r->enc = kb.first;
        r->mac = kb.second;
        r->slots.assign(staged_slots.begin(), staged_slots.end());
        r->key = k;
        r->last_seq = base_sequence_nonce + (n - 1);
        try {
            kr->inflight[{k, gen}].push_back(r);
            used.insert(staged.begin(), staged.end());
            if (r->last_seq > kr->get(kr->session_max, k)) kr->session_max[k] = r->last_seq;
        } catch (...) {
            kr->unlink(r);
            r->zeroize();
            delete r;
            throw;
        }
        *out = r;
        return 0;
    });
}

int ztcp_keyring_begin_egress(ztcp_keyring* kr, const char* tenant, const char* session, ztcp_reservation* res,
                              uint8_t enc_key[32], uint8_t mac_key[32]) {
    return guarded(kr, [&] {
        if (!strings_ok(tenant, session) || !res) throw Error{ZTCP_KR_EINVAL, "invalid argument"};
        const Key k{tenant, session};
        kr->check_reservation(k, res, "before or during egress");
        if (!nonzero(res->enc) || !nonzero(res->mac)) {
            res->zeroize();
            throw Error{ZTCP_KR_ESHREDDED, "Session (" + k.first + ", " + k.second + ") generation " +
                                               std::to_string(res->generation) + " key buffer was zeroized"};
        }
        copy_out(res->enc, enc_key);
        copy_out(res->mac, mac_key);
        return 0;
    });
}

int ztcp_keyring_commit_egress(ztcp_keyring* kr, const char* tenant, const char* session, ztcp_reservation* res) {
    return guarded(kr, [&] {
        if (!strings_ok(tenant, session) || !res) throw Error{ZTCP_KR_EINVAL, "invalid argument"};
        const Key k{tenant, session};
        kr->check_reservation(k, res, "before commit");
        auto& marks = kr->slot_latest[k];
        for (const auto& sv : res->slots) {
            auto m = marks.find(sv.first);
            if (m == marks.end()) marks.emplace(sv.first, sv.second);
            else if (sv.second > m->second) m->second = sv.second;
        }
        if (res->last_seq > kr->get(kr->session_max, k)) kr->session_max[k] = res->last_seq;
        return 0;
    });
}

void ztcp_keyring_release_reservation(ztcp_keyring* kr, const char* tenant, const char* session,
                                      ztcp_reservation* res) {
    (void)tenant;
    (void)session;
    if (!res) return;
    if (!kr) {
        res->zeroize();
        delete res;
        return;
    }
    std::lock_guard<std::mutex> lock(kr->mu);
    res->zeroize();
    kr->unlink(res);
    delete res;
}

uint64_t ztcp_reservation_last_sequence(const ztcp_reservation* res) { return res ? res->last_seq : 0; }

uint64_t ztcp_reservation_generation(const ztcp_reservation* res) { return res ? res->generation : 0; }

int ztcp_keyring_begin_ingress(ztcp_keyring* kr, const char* tenant, const char* session, uint64_t* generation,
                               uint8_t enc_key[32], uint8_t mac_key[32]) {
    return guarded(kr, [&] {
        if (!strings_ok(tenant, session)) throw Error{ZTCP_KR_EINVAL, "invalid argument"};
        const Key k{tenant, session};
        if (!kr->active.count(k))
            throw Error{ZTCP_KR_ESHREDDED, "Session (" + k.first + ", " + k.second + ") key is missing or crypto-shredded"};
        const uint64_t gen = kr->ensure_active(k);
        const auto& kb = kr->active.at(k);
        copy_out(kb.first, enc_key);
        copy_out(kb.second, mac_key);
        if (generation) *generation = gen;
        return 0;
    });
}

namespace {

void check_ingress_generation(ztcp_keyring* kr, const Key& k, const uint64_t* expected_generation) {
    if (!kr->active.count(k))
        throw Error{ZTCP_KR_ESHREDDED, "Session (" + k.first + ", " + k.second + ") key is missing or crypto-shredded"};
    const uint64_t cur = kr->ensure_active(k);
    if (expected_generation && (cur != *expected_generation || kr->get(kr->shredded_gen, k) >= *expected_generation))
        throw Error{ZTCP_KR_ESHREDDED, "Session (" + k.first + ", " + k.second + ") generation " +
                                           std::to_string(*expected_generation) + " was crypto-shredded during ingress"};
}

}  // namespace

int ztcp_keyring_verify_freshness(ztcp_keyring* kr, const char* tenant, const char* session, uint32_t model_id_hash,
                                  uint16_t layer_id, uint16_t head_group_id, uint64_t page_token_hash,
                                  uint64_t sequence_nonce, const uint64_t* min_sequence_nonce,
                                  const uint64_t* expected_sequence_nonce, const uint64_t* expected_generation) {
    return guarded(kr, [&] {
        if (!strings_ok(tenant, session)) throw Error{ZTCP_KR_EINVAL, "invalid argument"};
        const Key k{tenant, session};
        check_ingress_generation(kr, k, expected_generation);
        const uint64_t seq = sequence_nonce;
        if (expected_sequence_nonce && seq != *expected_sequence_nonce)
            throw Error{ZTCP_KR_ESTALE, "STALE_PAGE_REPLAY: Cold-page sequence_nonce=" + std::to_string(seq) +
                                            " != expected_sequence_nonce=" + std::to_string(*expected_sequence_nonce)};
        if (min_sequence_nonce && seq < *min_sequence_nonce)
            throw Error{ZTCP_KR_ESTALE, "STALE_PAGE_REPLAY: Cold-page sequence_nonce=" + std::to_string(seq) +
                                            " < min_sequence_nonce=" + std::to_string(*min_sequence_nonce)};
        auto& marks = kr->slot_latest[k];
        const Slot s{model_id_hash, layer_id, head_group_id, page_token_hash};
        auto m = marks.find(s);
        const uint64_t latest = m == marks.end() ? 0 : m->second;
        if (seq < latest)
            throw Error{ZTCP_KR_ESTALE, "STALE_PAGE_REPLAY: Cold-page sequence_nonce=" + std::to_string(seq) +
                                            " is older than latest slot version=" + std::to_string(latest)};
        if (seq > latest) marks[s] = seq;
        if (seq > kr->get(kr->session_max, k)) kr->session_max[k] = seq;
        return 0;
    });
}

int ztcp_keyring_verify_freshness_batch(ztcp_keyring* kr, const char* tenant, const char* session,
                                        const ztcp_freshness_record* records, size_t n,
                                        const uint64_t* min_sequence_nonce, const uint64_t* expected_generation) {
    return guarded(kr, [&] {
        if (!strings_ok(tenant, session) || (!records && n)) throw Error{ZTCP_KR_EINVAL, "invalid argument"};
        const Key k{tenant, session};
        check_ingress_generation(kr, k, expected_generation);
        auto& marks = kr->slot_latest[k];
        uint64_t max_s = kr->get(kr->session_max, k);
        std::unordered_map<Slot, uint64_t, SlotHash> staged;
        staged.reserve(n * 2);
        for (size_t i = 0; i < n; ++i) {
            const ztcp_freshness_record& r = records[i];
            const uint64_t seq = r.sequence_nonce;
            if (min_sequence_nonce && seq < *min_sequence_nonce)
                throw Error{ZTCP_KR_ESTALE, "STALE_PAGE_REPLAY: Cold-page sequence_nonce=" + std::to_string(seq) +
                                                " < min_sequence_nonce=" + std::to_string(*min_sequence_nonce)};
            const Slot s{r.model_id_hash, r.layer_id, r.head_group_id, r.page_token_hash};
            uint64_t latest = 0;
            auto st = staged.find(s);
            if (st != staged.end()) {
                latest = st->second;
            } else {
                auto m = marks.find(s);
                if (m != marks.end()) latest = m->second;
            }
            if (seq < latest)
                throw Error{ZTCP_KR_ESTALE, "STALE_PAGE_REPLAY: Cold-page sequence_nonce=" + std::to_string(seq) +
                                                " is older than latest slot version=" + std::to_string(latest)};
            if (seq > latest) staged[s] = seq;
            if (seq > max_s) max_s = seq;
        }
        for (const auto& sv : staged) marks[sv.first] = sv.second;
        kr->session_max[k] = max_s;
        return 0;
    });
}

int ztcp_keyring_finish_ingress(ztcp_keyring* kr, const char* tenant, const char* session,
                                uint64_t expected_generation) {
    return guarded(kr, [&] {
        if (!strings_ok(tenant, session)) throw Error{ZTCP_KR_EINVAL, "invalid argument"};
        const Key k{tenant, session};
        if (!kr->active.count(k) || kr->get(kr->session_gen, k) != expected_generation ||
            kr->get(kr->shredded_gen, k) >= expected_generation)
            throw Error{ZTCP_KR_ESHREDDED, "Session (" + k.first + ", " + k.second + ") generation " +
                                               std::to_string(expected_generation) +
                                               " was crypto-shredded during ingress"};
        return 0;
    });
}

int ztcp_keyring_shred_session(ztcp_keyring* kr, const char* tenant, const char* session) {
    return guarded(kr, [&] {
        if (!strings_ok(tenant, session)) throw Error{ZTCP_KR_EINVAL, "invalid argument"};
        return kr->shred(Key{tenant, session}) ? 1 : 0;
    });
}

int ztcp_keyring_shred_tenant(ztcp_keyring* kr, const char* tenant) {
    return guarded(kr, [&] {
        if (!tenant) throw Error{ZTCP_KR_EINVAL, "invalid argument"};
        std::vector<Key> keys;
        for (const auto& kv : kr->active)
            if (kv.first.first == tenant) keys.push_back(kv.first);
        for (const Key& k : keys) kr->shred(k);
        return (int)keys.size();
    });
}

const char* ztcp_keyring_last_error(void) { return t_last_error.c_str(); }

void ztcp_sha256(const uint8_t* data, size_t len, uint8_t out[32]) {
    Sha256 s;
    s.update(data, len);
    s.final(out);
}

void ztcp_hmac_sha256(const uint8_t* key, size_t key_len, const uint8_t* data, size_t len, uint8_t out[32]) {
    hmac_sha256(key, key_len, data, len, nullptr, 0, out);
}

}  // extern "C"
