// vib3file.cpp — host-side reader of the reference's `.vib3` model file (format.rs) and the
// builder of the fused layer's page table from it (engine.rs:1236-1299, generalised to several
// pages per segment). Host code only: the file is memory-mapped read-only, nothing touches the
// GPU, and the caller uploads pages and the table wherever it keeps them.
//
// On-disk layout (format.rs:9-26, :48-140; all structures little-endian and packed):
//   header (512 B) | model metadata (JSON) | page catalog (48 B entries, sorted by
//   (layer, expert, segment, page_idx)) | expert index (20 B entries) | ... | page data (2 MiB
//   aligned section, each page 4 KiB aligned).
#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <new>
#include <unordered_map>
#include <vector>

#include "../../include/vib3_hip.h"

namespace {

constexpr uint64_t kMagic = 0x3342495600000001ull;  // format.rs:39 VIB3_MAGIC
constexpr uint32_t kVersion = 1;
constexpr size_t kHeaderSize = 512;
constexpr size_t kCatalogEntry = 48;
constexpr size_t kExpertEntry = 20;

template <typename T>
T rd(const uint8_t* p) {
  T v;
  memcpy(&v, p, sizeof(T));
  return v;
}

struct ExpertRange {
  uint32_t first, count;
};

}  // namespace

struct vib3_file {
  int fd = -1;
  const uint8_t* map = nullptr;
  size_t size = 0;
  vib3_file_info info{};
  const uint8_t* metadata = nullptr;
  size_t metadata_size = 0;
  std::vector<vib3_page_entry> catalog;
  std::unordered_map<uint32_t, ExpertRange> experts;  // layer << 16 | expert
};

namespace {

// Header fields at their packed offsets (format.rs:50-92).
int parse(vib3_file* f) {
  const uint8_t* h = f->map;
  if (f->size < kHeaderSize) return VIB3_ERR_FORMAT;
  if (rd<uint64_t>(h + 0) != kMagic || rd<uint32_t>(h + 8) != kVersion) return VIB3_ERR_FORMAT;
  const uint64_t meta_off = rd<uint64_t>(h + 16), meta_size = rd<uint64_t>(h + 24);
  const uint64_t cat_off = rd<uint64_t>(h + 32);
  const uint32_t cat_count = rd<uint32_t>(h + 48);
  const uint64_t ei_off = rd<uint64_t>(h + 52), ei_size = rd<uint64_t>(h + 60);
  vib3_file_info& in = f->info;
  in.page_data_offset = rd<uint64_t>(h + 120);
  in.page_data_size = rd<uint64_t>(h + 128);
  in.num_layers = rd<uint32_t>(h + 136);
  in.num_experts = rd<uint32_t>(h + 140);
  in.num_active_experts = rd<uint32_t>(h + 144);
  in.hidden_dim = rd<uint32_t>(h + 148);
  in.expert_hidden_dim = rd<uint32_t>(h + 152);
  in.expert_dtype = h[156];
  in.shared_dtype = h[157];
  in.page_count = cat_count;
  if (meta_off > f->size || meta_size > f->size - meta_off) return VIB3_ERR_FORMAT;
  f->metadata = h + meta_off;
  f->metadata_size = (size_t)meta_size;
  if (cat_off > f->size || (uint64_t)cat_count * kCatalogEntry > f->size - cat_off)
    return VIB3_ERR_FORMAT;
  f->catalog.resize(cat_count);
  for (uint32_t i = 0; i < cat_count; i++) {
    const uint8_t* e = h + cat_off + (size_t)i * kCatalogEntry;  // format.rs:101-125
    vib3_page_entry& p = f->catalog[i];
    p.layer = rd<uint16_t>(e + 0);
    p.expert = rd<uint16_t>(e + 2);
    p.segment = rd<uint16_t>(e + 4);
    p.page_idx = rd<uint16_t>(e + 6);
    p.file_offset = rd<uint64_t>(e + 8);
    p.compressed_size = rd<uint32_t>(e + 16);
    p.raw_size = rd<uint32_t>(e + 20);
    p.row_start = rd<uint16_t>(e + 24);
    p.row_count = rd<uint16_t>(e + 26);
    p.col_start = rd<uint16_t>(e + 28);
    p.col_count = rd<uint16_t>(e + 30);
    p.compression = e[42];
    p.flags = e[43];
    p.catalog_index = i;
  }
  // expert index (format.rs:144-154); an absent or truncated section leaves it empty, as the
  // reference reader does (format.rs:286-291)
  if (ei_off <= f->size && ei_size <= f->size - ei_off && ei_size > 0) {
    const size_t n = (size_t)(ei_size / kExpertEntry);
    for (size_t i = 0; i < n; i++) {
      const uint8_t* e = h + ei_off + i * kExpertEntry;
      const uint32_t key = (uint32_t)rd<uint16_t>(e + 0) << 16 | rd<uint16_t>(e + 2);
      f->experts[key] = ExpertRange{rd<uint32_t>(e + 4), rd<uint32_t>(e + 8)};
    }
  }
  return 0;
}

}  // namespace

extern "C" {

int vib3_file_open(const char* path, vib3_file** out) {
  if (!path || !out) return VIB3_ERR_BAD_POINTER;
  *out = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return VIB3_ERR_IO;
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    close(fd);
    return VIB3_ERR_IO;
  }
  void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  if (m == MAP_FAILED) {
    close(fd);
    return VIB3_ERR_IO;
  }
  vib3_file* f = new (std::nothrow) vib3_file;
  if (!f) {
    munmap(m, (size_t)st.st_size);
    close(fd);
    return VIB3_ERR_IO;
  }
  f->fd = fd;
  f->map = (const uint8_t*)m;
  f->size = (size_t)st.st_size;
  const int rc = parse(f);
  if (rc) {
    vib3_file_close(f);
    return rc;
  }
  *out = f;
  return 0;
}

void vib3_file_close(vib3_file* f) {
  if (!f) return;
  if (f->map) munmap((void*)f->map, f->size);
  if (f->fd >= 0) close(f->fd);
  delete f;
}

int vib3_file_get_info(const vib3_file* f, vib3_file_info* info) {
  if (!f || !info) return VIB3_ERR_BAD_POINTER;
  *info = f->info;
  return 0;
}

int vib3_file_metadata(const vib3_file* f, const char** json, size_t* len) {
  if (!f || !json || !len) return VIB3_ERR_BAD_POINTER;
  *json = (const char*)f->metadata;
  *len = f->metadata_size;
  return 0;
}

int vib3_file_page(const vib3_file* f, uint32_t index, vib3_page_entry* entry) {
  if (!f || !entry) return VIB3_ERR_BAD_POINTER;
  if (index >= f->catalog.size()) return VIB3_ERR_BAD_COUNT;
  *entry = f->catalog[index];
  return 0;
}

int vib3_file_expert_pages(const vib3_file* f, uint16_t layer, uint16_t expert,
                           vib3_page_entry* out, int max_entries, int* count) {
  if (!f || !count || (max_entries > 0 && !out)) return VIB3_ERR_BAD_POINTER;
  *count = 0;
  auto it = f->experts.find((uint32_t)layer << 16 | expert);
  if (it == f->experts.end()) return 0;
  const ExpertRange r = it->second;
  if ((uint64_t)r.first + r.count > f->catalog.size()) return VIB3_ERR_FORMAT;
  *count = (int)r.count;
  for (uint32_t i = 0; i < r.count && (int)i < max_entries; i++) out[i] = f->catalog[r.first + i];
  return 0;
}

int vib3_file_page_data(const vib3_file* f, uint32_t index, const void** data, size_t* size) {
  if (!f || !data || !size) return VIB3_ERR_BAD_POINTER;
  if (index >= f->catalog.size()) return VIB3_ERR_BAD_COUNT;
  const vib3_page_entry& p = f->catalog[index];
  // LZ4 / zstd pages need the codec the reference links (lz4_flex, zstd); this build reads
  // uncompressed pages only (format.rs:501-565, the COMPRESSION_NONE arm)
  if (p.compression != 0) return VIB3_ERR_UNSUPPORTED;
  if (p.file_offset > f->size || p.compressed_size > f->size - p.file_offset)
    return VIB3_ERR_FORMAT;
  *data = f->map + p.file_offset;
  *size = p.compressed_size;
  return 0;
}

// LZ4 block decompression of lz4_flex's size-prepended frame (format.rs:526-533): a 4-byte
// little-endian decompressed size, then LZ4 sequences: a token (literal count in the high
// nibble, match length - 4 in the low one, 15 = more bytes follow, each adding up to 255),
// the literals, a 2-byte little-endian match offset and the extra match-length bytes; the
// last sequence has literals only. Every read and write is bounds-checked.
static int lz4_decompress(const uint8_t* src, size_t n, uint8_t* dst, size_t cap,
                          size_t* written) {
  if (n < 4) return VIB3_ERR_FORMAT;
  const size_t want = (size_t)rd<uint32_t>(src);
  if (want > cap) return VIB3_ERR_BAD_COUNT;
  size_t i = 4, o = 0;
  auto extend = [&](size_t& len) {
    uint8_t b;
    do {
      if (i >= n) return false;
      b = src[i++];
      len += b;
    } while (b == 255);
    return true;
  };
  while (i < n) {
    const uint8_t token = src[i++];
    size_t lit = token >> 4;
    if (lit == 15 && !extend(lit)) return VIB3_ERR_FORMAT;
    if (lit > n - i || lit > want - o) return VIB3_ERR_FORMAT;
    memcpy(dst + o, src + i, lit);
    i += lit;
    o += lit;
    if (i == n) break;  // the last sequence: literals only
    if (n - i < 2) return VIB3_ERR_FORMAT;
    const size_t off = rd<uint16_t>(src + i);
    i += 2;
    size_t len = (token & 15);
    if (len == 15 && !extend(len)) return VIB3_ERR_FORMAT;
    len += 4;
    if (off == 0 || off > o || len > want - o) return VIB3_ERR_FORMAT;
    for (size_t k = 0; k < len; k++, o++) dst[o] = dst[o - off];  // may overlap itself
  }
  if (o != want) return VIB3_ERR_FORMAT;
  *written = o;
  return 0;
}

int vib3_file_read_page(const vib3_file* f, uint32_t index, void* dst, size_t capacity,
                        size_t* written) {
  if (!f || !dst || !written) return VIB3_ERR_BAD_POINTER;
  if (index >= f->catalog.size()) return VIB3_ERR_BAD_COUNT;
  const vib3_page_entry& p = f->catalog[index];
  if (p.file_offset > f->size || p.compressed_size > f->size - p.file_offset)
    return VIB3_ERR_FORMAT;
  const uint8_t* src = f->map + p.file_offset;
  if (p.compression == 0) {  // COMPRESSION_NONE
    const size_t n = p.compressed_size < capacity ? p.compressed_size : capacity;
    memcpy(dst, src, n);
    *written = n;
    return 0;
  }
  if (p.compression == 1)  // COMPRESSION_LZ4
    return lz4_decompress(src, p.compressed_size, (uint8_t*)dst, capacity, written);
  return VIB3_ERR_UNSUPPORTED;  // zstd: no codec in this build
}

}  // extern "C"

namespace {

// One page of one (expert, segment) on its way into the table.
struct TablePage {
  uint32_t page_idx, row_start, row_count;
  uint64_t addr;
  uint32_t source;  // index in the caller's list (catalog index or resolved-page index)
};

// Writes table row (i, s) from the pages of one segment and checks that they are what the
// kernels address: page p holds rows [p * rpp, ...), every page but the last holds rpp rows
// (convert.rs:1852-1865), pages are distinct and gap-free, and together they cover
// rows_required rows (a truncated segment would leave the kernels reading address 0).
// Pages whose address is 0 are not resident: they are appended to `missing` and make the
// call return VIB3_ERR_NOT_RESIDENT once every other check has passed.
int fill_segment(std::vector<TablePage>& pages, int i, int s, int rows_required, int max_pages,
                 uint64_t* table, int rpp[3], uint32_t* missing, int max_missing,
                 int* n_missing) {
  if (pages.empty()) return VIB3_ERR_FORMAT;
  std::sort(pages.begin(), pages.end(),
            [](const TablePage& a, const TablePage& b) { return a.page_idx < b.page_idx; });
  int covered = 0;
  for (size_t j = 0; j < pages.size(); j++) {
    const TablePage& p = pages[j];
    if (p.page_idx >= (uint32_t)max_pages) return VIB3_ERR_BAD_COUNT;
    if (p.page_idx != j) return VIB3_ERR_FORMAT;  // a gap or the same page twice
    if (rpp[s] == 0 && p.page_idx == 0) rpp[s] = (int)p.row_count;
    if (rpp[s] == 0 || p.row_count == 0 || p.row_start != p.page_idx * (uint32_t)rpp[s] ||
        p.row_count > (uint32_t)rpp[s])
      return VIB3_ERR_FORMAT;
    if (j + 1 < pages.size() && p.row_count != (uint32_t)rpp[s])
      return VIB3_ERR_FORMAT;  // only the last page may be short
    covered = (int)(p.row_start + p.row_count);
    table[((size_t)i * 3 + s) * max_pages + p.page_idx] = p.addr;
    if (!p.addr) {
      if (*n_missing < max_missing && missing) missing[*n_missing] = p.source;
      (*n_missing)++;
    }
  }
  if (rows_required > 0 && covered < rows_required) return VIB3_ERR_FORMAT;
  return 0;
}

// Rows each segment must cover: the caller's, else the file's dimensions (gate/up rows =
// expert_hidden_dim, down rows = hidden_dim); 0 = unchecked (no file, no caller value).
void required_rows(const vib3_file* f, const int* rows_required, int out[3]) {
  for (int s = 0; s < 3; s++) {
    out[s] = rows_required ? rows_required[s] : 0;
    if (!rows_required && f)
      out[s] = (int)(s == 2 ? f->info.hidden_dim : f->info.expert_hidden_dim);
  }
}

}  // namespace

extern "C" {

int vib3_build_page_table(const vib3_file* f, uint16_t layer, const uint16_t* experts,
                          int num_experts, const uint16_t segments[3],
                          const uint64_t* page_addr, uint64_t* table, int max_pages,
                          int rows_per_page[3], const int* rows_required) {
  if (!f || !experts || !segments || !page_addr || !table || !rows_per_page)
    return VIB3_ERR_BAD_POINTER;
  if (num_experts <= 0 || max_pages <= 0) return VIB3_ERR_BAD_COUNT;
  memset(table, 0, sizeof(uint64_t) * (size_t)num_experts * 3 * max_pages);
  int rpp[3] = {0, 0, 0}, need[3];
  required_rows(f, rows_required, need);
  int n_missing = 0;
  for (int i = 0; i < num_experts; i++) {
    auto it = f->experts.find((uint32_t)layer << 16 | experts[i]);
    if (it == f->experts.end()) return VIB3_ERR_FORMAT;
    const ExpertRange r = it->second;
    const uint64_t qend = std::min<uint64_t>((uint64_t)r.first + r.count, f->catalog.size());
    for (int s = 0; s < 3; s++) {
      std::vector<TablePage> pages;
      for (uint64_t q = r.first; q < qend; q++) {
        const vib3_page_entry& p = f->catalog[q];
        if (p.segment == segments[s])
          pages.push_back({p.page_idx, p.row_start, p.row_count, page_addr[q], (uint32_t)q});
      }
      const int rc = fill_segment(pages, i, s, need[s], max_pages, table, rpp, nullptr, 0,
                                  &n_missing);
      if (rc) return rc;
    }
  }
  if (n_missing) return VIB3_ERR_NOT_RESIDENT;  // a page of the table has no address
  for (int s = 0; s < 3; s++) rows_per_page[s] = rpp[s];
  return 0;
}

int vib3_build_page_table_resolved(const vib3_resolved_page* pages, size_t num_pages,
                                   const uint16_t* experts, int num_experts,
                                   const uint16_t segments[3], const int rows_required[3],
                                   uint64_t* table, int max_pages, int rows_per_page[3],
                                   uint32_t* missing, int max_missing, int* num_missing) {
  if ((!pages && num_pages) || !experts || !segments || !table || !rows_per_page ||
      !num_missing || (max_missing > 0 && !missing))
    return VIB3_ERR_BAD_POINTER;
  if (num_experts <= 0 || max_pages <= 0 || max_missing < 0) return VIB3_ERR_BAD_COUNT;
  *num_missing = 0;
  memset(table, 0, sizeof(uint64_t) * (size_t)num_experts * 3 * max_pages);
  // (expert, segment) -> its pages, in one pass over the plan
  std::unordered_map<uint32_t, std::vector<TablePage>> by_key;
  for (size_t q = 0; q < num_pages; q++) {
    const vib3_resolved_page& p = pages[q];
    if (p.layer != pages[0].layer) return VIB3_ERR_FORMAT;  // one layer per table
    by_key[(uint32_t)p.expert << 16 | p.segment].push_back(
        {p.page_idx, p.row_start, p.row_count, p.device_ptr, (uint32_t)q});
  }
  int rpp[3] = {0, 0, 0}, need[3];
  required_rows(nullptr, rows_required, need);
  for (int i = 0; i < num_experts; i++) {
    for (int s = 0; s < 3; s++) {
      auto it = by_key.find((uint32_t)experts[i] << 16 | segments[s]);
      if (it == by_key.end()) return VIB3_ERR_FORMAT;
      const int rc = fill_segment(it->second, i, s, need[s], max_pages, table, rpp, missing,
                                  max_missing, num_missing);
      if (rc) return rc;
    }
  }
  for (int s = 0; s < 3; s++) rows_per_page[s] = rpp[s];
  return *num_missing ? VIB3_ERR_NOT_RESIDENT : 0;
}

}  // extern "C"
