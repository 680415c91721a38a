// zg_smodel.hip -- host-side reader of SilicatePack native .smodel files.
//
// Restates the reference loader's container checks and SIDX index walk
// (kernel/src/model_loader.rs: constants :38-79, smodel_decode_dtype
// :82-90, smodel_native_tensor_index :380-575, smodel_info :599-659) over
// a caller-owned byte image, so that a packed artifact enters the same
// registry and model path as the rest of the library.  The layout written
// by the packer is tools/silicatepack.py:266-294 (header) and :1097-1161
// (SIDX).  Host code only.
#include <stdint.h>
#include <string.h>

#include <new>
#include <vector>

#include "../../include/zero_gpu.h"

namespace {

constexpr uint32_t kMagicSilm = 0x4D4C4953;  // "SILM"
constexpr uint32_t kMagicSidx = 0x58444953;  // "SIDX"
constexpr size_t kHeaderSize = 128;
constexpr size_t kIndexHeaderSize = 128;
constexpr size_t kEntrySize = 104;
constexpr size_t kMaxTensors = 10000;
constexpr uint64_t kPayloadAlignment = 2ull * 1024 * 1024;
constexpr uint32_t kKindGgufCompat = 1, kKindNative = 2;
constexpr uint32_t kDtypeQ4_0X4 = 100, kDtypeQ8_0X4 = 101;

// Little-endian reads with bounds (read_u32_le / read_u64_le, model_loader.rs:162-197).
bool rd32(const uint8_t* b, size_t len, size_t off, uint32_t& v) {
  if (off > len || len - off < 4) return false;
  v = (uint32_t)b[off] | ((uint32_t)b[off + 1] << 8) | ((uint32_t)b[off + 2] << 16) | ((uint32_t)b[off + 3] << 24);
  return true;
}
bool rd64(const uint8_t* b, size_t len, size_t off, uint64_t& v) {
  uint32_t lo, hi;
  if (!rd32(b, len, off, lo) || !rd32(b, len, off + 4, hi)) return false;
  v = (uint64_t)lo | ((uint64_t)hi << 32);
  return true;
}
bool rdf32(const uint8_t* b, size_t len, size_t off, float& v) {
  uint32_t u;
  if (!rd32(b, len, off, u)) return false;
  memcpy(&v, &u, 4);
  return true;
}
bool add_ok(uint64_t a, uint64_t b, uint64_t& r) {
  r = a + b;
  return r >= a;
}

// GgmlType::from_u32 (crates/zero-gguf-parser/src/lib.rs:129-162): 0..3, 6..30.
bool ggml_type_known(uint32_t t) { return t <= 3 || (t >= 6 && t <= 30); }

// smodel_decode_dtype (model_loader.rs:82-90).
bool decode_dtype(uint32_t dtype, uint32_t& ggml, uint32_t& interleave) {
  if (dtype == kDtypeQ4_0X4) {
    ggml = ZG_Q4_0;
    interleave = 4;
    return true;
  }
  if (dtype == kDtypeQ8_0X4) {
    ggml = ZG_Q8_0;
    interleave = 4;
    return true;
  }
  if (!ggml_type_known(dtype)) return false;
  ggml = dtype;
  interleave = 1;
  return true;
}

// Strict UTF-8 check (core::str::from_utf8 semantics: no overlongs, no
// surrogates, at most U+10FFFF).
bool valid_utf8(const uint8_t* s, size_t n) {
  size_t i = 0;
  while (i < n) {
    const uint8_t c = s[i];
    if (c < 0x80) {
      i++;
      continue;
    }
    size_t len;
    uint32_t cp;
    if ((c & 0xE0) == 0xC0) {
      len = 2;
      cp = c & 0x1F;
    } else if ((c & 0xF0) == 0xE0) {
      len = 3;
      cp = c & 0x0F;
    } else if ((c & 0xF8) == 0xF0) {
      len = 4;
      cp = c & 0x07;
    } else {
      return false;
    }
    if (n - i < len) return false;
    for (size_t k = 1; k < len; k++) {
      if ((s[i + k] & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (s[i + k] & 0x3F);
    }
    if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000)) return false;
    if (cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
    i += len;
  }
  return true;
}

}  // namespace

struct zg_smodel {
  const uint8_t* bytes = nullptr;
  size_t len = 0;
  zg_smodel_info info{};
  std::vector<zg_smodel_tensor> tensors;
};

extern "C" zg_status zg_smodel_open(const void* bytes_v, size_t len, zg_smodel** out) {
  if (!bytes_v || !out) return ZG_ERR_INVALID_ARG;
  *out = nullptr;
  const uint8_t* b = static_cast<const uint8_t*>(bytes_v);
  // smodel_info (model_loader.rs:599-659)
  if (len < kHeaderSize) return ZG_ERR_INVALID_CONTAINER;
  uint32_t magic = 0;
  rd32(b, len, 0, magic);
  if (magic != kMagicSilm) return ZG_ERR_MAGIC_MISMATCH;
  zg_smodel_info info{};
  uint32_t header_len = 0;
  rd32(b, len, 4, info.version);
  if (info.version != 1 && info.version != 2) return ZG_ERR_UNSUPPORTED_FORMAT;
  rd32(b, len, 8, header_len);
  rd64(b, len, 12, info.manifest_offset);
  rd64(b, len, 20, info.manifest_len);
  rd64(b, len, 28, info.payload_offset);
  rd64(b, len, 36, info.payload_len);
  rd32(b, len, 44, info.payload_kind);
  rd32(b, len, 48, info.flags);
  if (header_len != kHeaderSize) return ZG_ERR_UNSUPPORTED_FORMAT;
  if (info.payload_kind != kKindGgufCompat && info.payload_kind != kKindNative) return ZG_ERR_UNSUPPORTED_FORMAT;
  if (info.manifest_len == 0) return ZG_ERR_INVALID_CONTAINER;
  uint64_t manifest_end, payload_end;
  if (!add_ok(info.manifest_offset, info.manifest_len, manifest_end) ||
      !add_ok(info.payload_offset, info.payload_len, payload_end))
    return ZG_ERR_INVALID_CONTAINER;
  if (info.manifest_offset < header_len || manifest_end > info.payload_offset || info.payload_offset < header_len ||
      payload_end > len || info.payload_len < 4)
    return ZG_ERR_INVALID_CONTAINER;
  if ((info.flags & 1) && info.payload_offset % kPayloadAlignment != 0) return ZG_ERR_INVALID_CONTAINER;
  if (info.payload_kind == kKindNative && info.payload_len < kIndexHeaderSize) return ZG_ERR_INVALID_CONTAINER;
  // the GGUF-compatibility payload is a wrapped GGUF: not a native index
  if (info.payload_kind != kKindNative) return ZG_ERR_UNSUPPORTED_FORMAT;

  // SIDX header (smodel_native_tensor_index, model_loader.rs:380-454)
  const uint8_t* p = b + info.payload_offset;
  const size_t plen = (size_t)info.payload_len;
  uint32_t sidx = 0, iver = 0, ihdr = 0, count = 0, entry_size = 0, names_offset = 0, names_len = 0;
  rd32(p, plen, 0, sidx);
  rd32(p, plen, 4, iver);
  rd32(p, plen, 8, ihdr);
  if (sidx != kMagicSidx || iver != 1 || ihdr != kIndexHeaderSize) return ZG_ERR_UNSUPPORTED_FORMAT;
  rd32(p, plen, 12, count);
  if (count > kMaxTensors) return ZG_ERR_INVALID_CONTAINER;
  rd32(p, plen, 16, entry_size);
  rd32(p, plen, 20, names_offset);
  rd32(p, plen, 24, names_len);
  if (entry_size != kEntrySize) return ZG_ERR_UNSUPPORTED_FORMAT;
  const uint64_t entries_end = kIndexHeaderSize + (uint64_t)count * kEntrySize;
  const uint64_t names_end = (uint64_t)names_offset + names_len;
  if (entries_end > plen || names_offset < entries_end || names_end > plen) return ZG_ERR_INVALID_CONTAINER;
  rd32(p, plen, 36, info.architecture_id);
  rd32(p, plen, 40, info.block_count);
  rd32(p, plen, 44, info.context_length);
  rd32(p, plen, 48, info.embedding_length);
  rd32(p, plen, 52, info.feed_forward_length);
  rd32(p, plen, 56, info.head_count);
  rd32(p, plen, 60, info.head_count_kv);
  rd32(p, plen, 64, info.key_length);
  rd32(p, plen, 68, info.value_length);
  rdf32(p, plen, 72, info.rope_freq_base);
  rdf32(p, plen, 76, info.layer_norm_rms_epsilon);
  rd32(p, plen, 80, info.vocab_size);
  rd32(p, plen, 84, info.eos_token_id);
  info.tensor_count = count;

  const uint8_t* names = p + names_offset;
  zg_smodel* sm = new (std::nothrow) zg_smodel;
  if (!sm) return ZG_ERR_OUT_OF_MEMORY;
  std::vector<zg_smodel_tensor>& tensors = sm->tensors;
  try {
    tensors.reserve(count);  // count <= kMaxTensors: no growth below
  } catch (const std::bad_alloc&) {  // no exception crosses the C ABI
    delete sm;
    return ZG_ERR_OUT_OF_MEMORY;
  }
  auto fail = [&](zg_status e) {
    delete sm;
    return e;
  };
  for (uint32_t i = 0; i < count; i++) {
    const size_t off = kIndexHeaderSize + (size_t)i * kEntrySize;
    uint32_t name_off = 0, name_len = 0, dtype = 0, rank = 0;
    rd32(p, plen, off, name_off);
    rd32(p, plen, off + 4, name_len);
    rd32(p, plen, off + 8, dtype);
    rd32(p, plen, off + 12, rank);
    if (rank > 8) return fail(ZG_ERR_INVALID_CONTAINER);
    const uint64_t name_end = (uint64_t)name_off + name_len;
    if (name_end > names_len || !valid_utf8(names + name_off, name_len)) return fail(ZG_ERR_INVALID_CONTAINER);
    zg_smodel_tensor t{};
    t.name = reinterpret_cast<const char*>(names + name_off);
    t.name_len = name_len;
    t.dtype = dtype;
    t.rank = rank;
    for (uint32_t d = 0; d < 8; d++) t.dims[d] = 1;
    for (uint32_t d = 0; d < rank; d++) rd64(p, plen, off + 16 + 8 * d, t.dims[d]);
    rd64(p, plen, off + 80, t.payload_offset);
    rd64(p, plen, off + 88, t.byte_len);
    uint64_t tensor_end;
    if (!add_ok(t.payload_offset, t.byte_len, tensor_end) || tensor_end > plen) return fail(ZG_ERR_INVALID_CONTAINER);
    if (!decode_dtype(dtype, t.ggml_type, t.interleave)) return fail(ZG_ERR_UNSUPPORTED_FORMAT);
    // interleaving needs a rank-2 matmul weight with rows % 4 == 0 (:527-544)
    if (t.interleave > 1 && !(rank == 2 && t.dims[0] % t.interleave == 0)) return fail(ZG_ERR_INVALID_CONTAINER);
    t.data = p + t.payload_offset;
    tensors.push_back(t);
  }
  sm->bytes = b;
  sm->len = len;
  sm->info = info;
  *out = sm;
  return ZG_OK;
}

extern "C" void zg_smodel_close(zg_smodel* sm) { delete sm; }

extern "C" zg_status zg_smodel_get_info(const zg_smodel* sm, zg_smodel_info* out) {
  if (!sm || !out) return ZG_ERR_INVALID_ARG;
  *out = sm->info;
  return ZG_OK;
}

extern "C" zg_status zg_smodel_get_tensor(const zg_smodel* sm, uint64_t index, zg_smodel_tensor* out) {
  if (!sm || !out || index >= sm->tensors.size()) return ZG_ERR_INVALID_ARG;
  *out = sm->tensors[index];
  return ZG_OK;
}

extern "C" zg_status zg_smodel_find(const zg_smodel* sm, const char* name, zg_smodel_tensor* out) {
  if (!sm || !name || !out) return ZG_ERR_INVALID_ARG;
  const size_t n = strlen(name);
  for (const zg_smodel_tensor& t : sm->tensors) {
    if (t.name_len == n && memcmp(t.name, name, n) == 0) {
      *out = t;
      return ZG_OK;
    }
  }
  return ZG_ERR_INVALID_ARG;
}

extern "C" zg_status zg_smodel_register_all(zg_ctx* ctx, const zg_smodel* sm) {
  if (!ctx || !sm) return ZG_ERR_INVALID_ARG;
  for (const zg_smodel_tensor& t : sm->tensors) {
    if (t.ggml_type != ZG_Q4_0 && t.ggml_type != ZG_Q8_0 && t.ggml_type != ZG_Q4K && t.ggml_type != ZG_Q6K) continue;
    const zg_status s = zg_register_weight(ctx, t.data, (size_t)t.byte_len, t.ggml_type, t.interleave);
    if (s) return s;
  }
  return ZG_OK;
}
