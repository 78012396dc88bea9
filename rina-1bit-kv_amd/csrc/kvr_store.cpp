// Host side of the tile-store file format declared in include/kvr_store.h: the header
// codec, the section layout and CRC-32.  No device code and no HIP call: a store is
// moved between device memory and a file by the caller (the Python layer copies each
// section), so these functions only define and check the bytes.
#include <cstdint>
#include <cstring>
#include <initializer_list>

#include "../../include/kvr_store.h"
#include "kvr_internal.h"

namespace {

constexpr char kMagic[8] = {'K', 'V', 'R', 'S', 'T', 'O', 'R', 'E'};
constexpr int64_t kMaxBytes = (int64_t)1 << 56;  // any section or payload larger is rejected

struct CrcTable {
  uint32_t t[256];
};
constexpr CrcTable make_crc_table() {
  CrcTable c{};
  for (uint32_t i = 0; i < 256; ++i) {
    uint32_t r = i;
    for (int b = 0; b < 8; ++b) r = (r & 1u) ? (r >> 1) ^ 0xEDB88320u : r >> 1;
    c.t[i] = r;
  }
  return c;
}
constexpr CrcTable kCrc = make_crc_table();

template <typename V>
void put(uint8_t* h, int off, V v) {
  std::memcpy(h + off, &v, sizeof(V));  // the host is little-endian (x86-64)
}
template <typename V>
V get(const uint8_t* h, int off) {
  V v;
  std::memcpy(&v, h + off, sizeof(V));
  return v;
}

int64_t elem_bytes(int dt) { return dt == KVR_FP32 ? 4 : 2; }
int64_t align_up(int64_t x) { return (x + KVR_STORE_ALIGN - 1) / KVR_STORE_ALIGN * KVR_STORE_ALIGN; }

// a * b * ..., or -1 past kMaxBytes
int64_t mul_checked(std::initializer_list<int64_t> xs) {
  int64_t p = 1;
  for (int64_t x : xs) {
    if (x < 0) return -1;
    if (x != 0 && p > kMaxBytes / x) return -1;
    p *= x;
  }
  return p;
}

int check_desc(const kvr_store_desc* s) {
  if (!s) return kvr::set_error(KVR_ERR_INVALID, "store description is NULL");
  if (s->d != 128) return kvr::set_error(KVR_ERR_INVALID, "store: d=%d unsupported (must be 128)", s->d);
  if (s->T != 64 && s->T != 128) return kvr::set_error(KVR_ERR_INVALID, "store: T=%d unsupported (64 or 128)", s->T);
  if (s->transform != KVR_HADAMARD && s->transform != KVR_DCT && s->transform != KVR_NONE)
    return kvr::set_error(KVR_ERR_INVALID, "store: transform %d unknown", s->transform);
  if (s->bit_order != KVR_BITS_TOKEN_LSB)
    return kvr::set_error(KVR_ERR_UNSUPPORTED, "store: bit order %d unknown", s->bit_order);
  if (s->scale_dtype != KVR_FP16) return kvr::set_error(KVR_ERR_UNSUPPORTED, "store: scale dtype %d unsupported", s->scale_dtype);
  if (s->flags & ~(uint32_t)(KVR_STORE_HAS_COUNTS | KVR_STORE_HAS_WINDOW))
    return kvr::set_error(KVR_ERR_UNSUPPORTED, "store: unknown flags 0x%x", s->flags);
  if (s->n_layers < 1) return kvr::set_error(KVR_ERR_INVALID, "store: n_layers=%d < 1", s->n_layers);
  if (s->B < 0 || s->Hkv < 1 || s->n_tiles < 0)
    return kvr::set_error(KVR_ERR_INVALID, "store: bad sizes B=%lld Hkv=%lld n_tiles=%lld", (long long)s->B,
                          (long long)s->Hkv, (long long)s->n_tiles);
  if (s->W < 0 || s->W % s->T)
    return kvr::set_error(KVR_ERR_INVALID, "store: W=%lld must be a non-negative multiple of T=%d", (long long)s->W, s->T);
  if (s->flags & KVR_STORE_HAS_WINDOW) {
    if (s->win_dtype != KVR_BF16 && s->win_dtype != KVR_FP16 && s->win_dtype != KVR_FP32)
      return kvr::set_error(KVR_ERR_INVALID, "store: window dtype %d unknown", s->win_dtype);
    if (s->win_len < 0 || s->win_len >= s->W + s->T)
      return kvr::set_error(KVR_ERR_INVALID, "store: win_len=%lld outside [0, W + T = %lld)", (long long)s->win_len,
                            (long long)(s->W + s->T));
  } else if (s->win_len != 0) {
    return kvr::set_error(KVR_ERR_INVALID, "store: win_len=%lld without a window section", (long long)s->win_len);
  }
  return KVR_OK;
}

// bytes of each section of one layer (0 for absent ones), -1 on overflow
bool section_sizes(const kvr_store_desc* s, int64_t (&sz)[KVR_SEC_N]) {
  const int64_t seg = mul_checked({s->B, s->Hkv});
  const int64_t tiles = mul_checked({seg, s->n_tiles});
  sz[KVR_SEC_KBITS] = sz[KVR_SEC_VBITS] = mul_checked({tiles, 128, (int64_t)(s->T / 64), 8});
  sz[KVR_SEC_KSCALE] = sz[KVR_SEC_VSCALE] = mul_checked({tiles, 2});
  sz[KVR_SEC_KCOUNT] = (s->flags & KVR_STORE_HAS_COUNTS) ? mul_checked({tiles, 128}) : 0;
  const bool win = (s->flags & KVR_STORE_HAS_WINDOW) != 0;
  sz[KVR_SEC_WIN_K] = sz[KVR_SEC_WIN_V] = win ? mul_checked({seg, s->win_len, 128, elem_bytes(s->win_dtype)}) : 0;
  for (int64_t v : sz)
    if (v < 0) return false;
  return seg >= 0 && tiles >= 0;
}

bool section_present(const kvr_store_desc* s, int sec) {
  if (sec == KVR_SEC_KCOUNT) return (s->flags & KVR_STORE_HAS_COUNTS) != 0;
  if (sec == KVR_SEC_WIN_K || sec == KVR_SEC_WIN_V) return (s->flags & KVR_STORE_HAS_WINDOW) != 0;
  return true;
}

// aligned bytes of one layer's sections (-1 on overflow)
int64_t layer_bytes(const kvr_store_desc* s) {
  int64_t sz[KVR_SEC_N];
  if (!section_sizes(s, sz)) return -1;
  int64_t t = 0;
  for (int i = 0; i < KVR_SEC_N; ++i) {
    if (!section_present(s, i)) continue;
    t += align_up(sz[i]);
    if (t > kMaxBytes) return -1;
  }
  return t;
}

}  // namespace

extern "C" {

uint32_t kvr_crc32(uint32_t crc, const void* data, size_t n) {
  const uint8_t* p = (const uint8_t*)data;
  uint32_t c = ~crc;
  for (size_t i = 0; i < n; ++i) c = kCrc.t[(c ^ p[i]) & 0xffu] ^ (c >> 8);
  return ~c;
}

int64_t kvr_store_payload_bytes(const kvr_store_desc* desc) {
  if (int r = check_desc(desc)) return r;
  const int64_t lb = layer_bytes(desc);
  if (lb < 0 || (lb > 0 && desc->n_layers > kMaxBytes / lb))
    return kvr::set_error(KVR_ERR_INVALID, "store: payload size overflows");
  return lb * desc->n_layers;
}

int64_t kvr_store_section(const kvr_store_desc* desc, int layer, int section, int64_t* bytes) {
  const int64_t total = kvr_store_payload_bytes(desc);
  if (total < 0) return total;
  if (layer < 0 || layer >= desc->n_layers)
    return kvr::set_error(KVR_ERR_INVALID, "store: layer %d outside [0, %d)", layer, desc->n_layers);
  if (section < 0 || section >= KVR_SEC_N) return kvr::set_error(KVR_ERR_INVALID, "store: section %d unknown", section);
  if (!section_present(desc, section))
    return kvr::set_error(KVR_ERR_INVALID, "store: section %d is not in this store (flags 0x%x)", section, desc->flags);
  int64_t sz[KVR_SEC_N];
  section_sizes(desc, sz);
  int64_t off = KVR_STORE_HEADER_BYTES + (int64_t)layer * layer_bytes(desc);
  for (int i = 0; i < section; ++i)
    if (section_present(desc, i)) off += align_up(sz[i]);
  if (bytes) *bytes = sz[section];
  return off;
}

int kvr_store_header_encode(const kvr_store_desc* desc, void* header) {
  if (!header) return kvr::set_error(KVR_ERR_INVALID, "store: header buffer is NULL");
  const int64_t payload = kvr_store_payload_bytes(desc);
  if (payload < 0) return (int)payload;
  uint8_t* h = (uint8_t*)header;
  std::memset(h, 0, KVR_STORE_HEADER_BYTES);
  std::memcpy(h, kMagic, 8);
  put<uint32_t>(h, 8, KVR_STORE_FORMAT_VERSION);
  put<uint32_t>(h, 12, KVR_STORE_HEADER_BYTES);
  put<uint32_t>(h, 16, (uint32_t)kvr_abi_version());
  put<int32_t>(h, 20, desc->d);
  put<int32_t>(h, 24, desc->T);
  put<int32_t>(h, 28, desc->transform);
  put<int32_t>(h, 32, desc->bit_order);
  put<int32_t>(h, 36, desc->scale_dtype);
  put<int32_t>(h, 40, (desc->flags & KVR_STORE_HAS_WINDOW) ? desc->win_dtype : 0);
  put<uint32_t>(h, 44, desc->flags);
  put<int32_t>(h, 48, desc->n_layers);
  put<uint32_t>(h, 52, KVR_STORE_ALIGN);
  put<int64_t>(h, 56, desc->B);
  put<int64_t>(h, 64, desc->Hkv);
  put<int64_t>(h, 72, desc->n_tiles);
  put<int64_t>(h, 80, desc->W);
  put<int64_t>(h, 88, desc->win_len);
  put<uint64_t>(h, 96, (uint64_t)payload);
  put<uint32_t>(h, 104, desc->payload_crc32);
  for (int i = 0; i < 4; ++i) put<int64_t>(h, 112 + 8 * i, desc->user[i]);
  put<uint32_t>(h, 252, kvr_crc32(0, h, 252));
  return KVR_OK;
}

int kvr_store_header_decode(const void* header, size_t n, kvr_store_desc* desc) {
  if (!header || !desc) return kvr::set_error(KVR_ERR_INVALID, "store: NULL header or description");
  if (n < KVR_STORE_HEADER_BYTES)
    return kvr::set_error(KVR_ERR_INVALID, "store: %zu header bytes, need %d", n, KVR_STORE_HEADER_BYTES);
  const uint8_t* h = (const uint8_t*)header;
  if (std::memcmp(h, kMagic, 8) != 0) return kvr::set_error(KVR_ERR_INVALID, "store: not a KVRSTORE file (bad magic)");
  const uint32_t version = get<uint32_t>(h, 8);
  if (version > KVR_STORE_FORMAT_VERSION || version == 0)
    return kvr::set_error(KVR_ERR_UNSUPPORTED, "store: format version %u (this library reads up to %d)", version,
                          KVR_STORE_FORMAT_VERSION);
  if (get<uint32_t>(h, 252) != kvr_crc32(0, h, 252))
    return kvr::set_error(KVR_ERR_INVALID, "store: header CRC mismatch (corrupted header)");
  if (get<uint32_t>(h, 12) != KVR_STORE_HEADER_BYTES || get<uint32_t>(h, 52) != KVR_STORE_ALIGN)
    return kvr::set_error(KVR_ERR_UNSUPPORTED, "store: header size %u / alignment %u unsupported", get<uint32_t>(h, 12),
                          get<uint32_t>(h, 52));
  kvr_store_desc s{};
  s.format_version = version;
  s.abi_version = get<uint32_t>(h, 16);
  s.d = get<int32_t>(h, 20);
  s.T = get<int32_t>(h, 24);
  s.transform = get<int32_t>(h, 28);
  s.bit_order = get<int32_t>(h, 32);
  s.scale_dtype = get<int32_t>(h, 36);
  s.win_dtype = get<int32_t>(h, 40);
  s.flags = get<uint32_t>(h, 44);
  s.n_layers = get<int32_t>(h, 48);
  s.B = get<int64_t>(h, 56);
  s.Hkv = get<int64_t>(h, 64);
  s.n_tiles = get<int64_t>(h, 72);
  s.W = get<int64_t>(h, 80);
  s.win_len = get<int64_t>(h, 88);
  s.payload_bytes = get<uint64_t>(h, 96);
  s.payload_crc32 = get<uint32_t>(h, 104);
  for (int i = 0; i < 4; ++i) s.user[i] = get<int64_t>(h, 112 + 8 * i);
  const int64_t payload = kvr_store_payload_bytes(&s);
  if (payload < 0) return (int)payload;
  if ((uint64_t)payload != s.payload_bytes)
    return kvr::set_error(KVR_ERR_INVALID, "store: header says %llu payload bytes, its fields give %lld",
                          (unsigned long long)s.payload_bytes, (long long)payload);
  *desc = s;
  return KVR_OK;
}

}  // extern "C"
