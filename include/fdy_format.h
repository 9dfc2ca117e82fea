/*
 * fdy_format.h -- the `.cugraph` v1 archive layout, as plain packed C structs.
 *
 * Byte-compatible with the reference's on-disk format so that archives written
 * by the reference's SAVE path restore here unchanged:
 *   include/BinaryGraphFormat.h:37-53   magic, version, section ids
 *   include/BinaryGraphFormat.h:55-61   header flags
 *   include/BinaryGraphFormat.h:65-84   FileHeader (64 B), SectionEntry (24 B)
 *   include/BinaryGraphFormat.h:88-185  node types and the 168-B node entry
 *   include/BinaryGraphFormat.h:189-227 param entry, common attrs, generator, dependency
 *   csrc/BinaryGraphIO.cpp:292-315      section order; every section starts 8-B aligned
 *   csrc/BinaryGraphIO.cpp:214          0xFFFFFFFF = "no extra arg buffer"
 *
 * The field layout has to match byte for byte; the names and the C spelling
 * are this library's own.  Everything is little-endian.  The node entry is
 * packed, so `kernel.binary_hash` sits at entry offset 36 (4-B aligned only):
 * device code reads it as two u32 halves.
 */
#ifndef FDY_FORMAT_H
#define FDY_FORMAT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FDY_MAGIC_0 0x43u /* 'C' */
#define FDY_FORMAT_VERSION 1u
#define FDY_NO_ARG_BUFFER 0xFFFFFFFFu

/* Section ids, in the order the writer lays them out. */
enum fdy_section_id {
  FDY_SEC_STRINGS = 0,
  FDY_SEC_NODES = 1,
  FDY_SEC_DEPS = 2,
  FDY_SEC_PARAM_INDEX = 3,
  FDY_SEC_PARAM_DATA = 4,
  FDY_SEC_ARG_DATA = 5,
  FDY_SEC_COMMON_ATTRS = 6,
  FDY_SEC_GENERATORS = 7,
  FDY_SEC_ALLOC_EVENTS = 8,
  FDY_SEC_OUTPUT_TENSORS = 9,
  FDY_SEC_TOPOLOGY_KEY = 10,
  FDY_SEC_COUNT = 11
};

enum fdy_header_flag {
  FDY_HAS_COMMON_ATTRS = 1u << 0,
  FDY_HAS_DEPS = 1u << 1,
  FDY_HAS_ALLOC_EVENTS = 1u << 2,
  FDY_HAS_OUTPUT_TENSORS = 1u << 3,
  FDY_HAS_GENERATORS = 1u << 4
};

enum fdy_node_type {
  FDY_NODE_KERNEL = 0,
  FDY_NODE_MEMSET = 1,
  FDY_NODE_MEMCPY = 2,
  FDY_NODE_EVENT_RECORD = 3,
  FDY_NODE_EVENT_WAIT = 4,
  FDY_NODE_EMPTY = 5
};

/* Which per-node launch attributes are present (kna_flags / common flags). */
enum fdy_kna_flag {
  FDY_KNA_CLUSTER_DIM = 1u << 0,
  FDY_KNA_PREFERRED_CLUSTER_DIM = 1u << 1,
  FDY_KNA_CLUSTER_SCHEDULING = 1u << 2,
  FDY_KNA_COOPERATIVE = 1u << 3,
  FDY_KNA_PRIORITY = 1u << 4,
  FDY_KNA_MEM_SYNC_DOMAIN = 1u << 5,
  FDY_KNA_MEM_SYNC_DOMAIN_MAP = 1u << 6,
  FDY_KNA_SHARED_MEM_CARVEOUT = 1u << 7,
  FDY_KNA_ATTR_QUERY_AVAILABLE = 1u << 8
};

#pragma pack(push, 1)

typedef struct fdy_file_header {
  uint8_t magic[8]; /* "CUGRAPH\0" */
  uint32_t version;
  uint32_t flags; /* fdy_header_flag */
  uint32_t num_nodes;
  uint32_t num_deps;
  uint32_t num_generators;
  uint32_t num_sections;
  uint32_t num_strings;
  uint8_t reserved[28];
} fdy_file_header;

typedef struct fdy_section {
  uint32_t id;
  uint32_t pad;
  uint64_t offset; /* from the start of the file */
  uint64_t size;   /* bytes */
} fdy_section;

typedef struct fdy_kernel_body {
  uint32_t block[3];
  uint32_t grid[3];
  uint32_t shared_mem_bytes;
  uint64_t binary_hash; /* CRC-64/XZ of the code object that holds the function */
  uint32_t name_offset; /* into the string section */
  uint32_t name_length;
  int32_t max_dynamic_shared;
  int32_t preferred_carveout;
  int32_t cluster_sched_pref;
  int32_t required_cluster[3];
  uint32_t kna_flags;
  uint32_t kna_cluster[3];
  uint32_t kna_preferred_cluster[3];
  int32_t kna_cluster_sched;
  int32_t kna_cooperative;
  int32_t kna_priority;
  int32_t kna_mem_sync_domain;
  uint8_t kna_mem_sync_map_default;
  uint8_t kna_mem_sync_map_remote;
  uint8_t kna_attr_query_available;
  uint8_t kna_pad;
  uint32_t kna_preferred_carveout;
  uint32_t param_index_offset; /* bytes into the param-index section */
  uint32_t num_params;
  uint32_t arg_offset; /* bytes into the arg section, or FDY_NO_ARG_BUFFER */
  uint32_t arg_size;
} fdy_kernel_body;

typedef struct fdy_memset_body {
  uint64_t dst;
  uint32_t element_size;
  uint32_t pad0;
  uint64_t height;
  uint64_t pitch;
  uint32_t value;
  uint32_t pad1;
  uint64_t width;
} fdy_memset_body;

typedef struct fdy_memcpy_body {
  uint64_t depth, height, width_bytes;
  uint64_t dst;
  uint64_t dst_height, dst_lod, dst_pitch, dst_x_bytes, dst_y, dst_z;
  int32_t dst_mem_type;
  int32_t pad0;
  uint64_t src;
  uint64_t src_height, src_lod, src_pitch, src_x_bytes, src_y, src_z;
  int32_t src_mem_type;
  int32_t pad1;
} fdy_memcpy_body;

typedef struct fdy_event_body {
  int32_t event_id;
} fdy_event_body;

typedef struct fdy_node {
  uint32_t node_id;
  uint8_t type; /* fdy_node_type */
  uint8_t pad[3];
  union {
    fdy_kernel_body kernel;
    fdy_memset_body memset;
    fdy_memcpy_body memcpy;
    fdy_event_body event;
    uint8_t raw[152];
  } u;
  uint8_t tail[8];
} fdy_node;

typedef struct fdy_param {
  uint32_t data_offset; /* bytes into the param-data section (extra-style: in-kernel offset) */
  uint32_t size;
} fdy_param;

typedef struct fdy_common_attrs {
  uint32_t flags; /* fdy_kna_flag: which attributes are common to every kernel node */
  uint32_t cluster[3];
  uint32_t preferred_cluster[3];
  int32_t cluster_sched;
  int32_t cooperative;
  int32_t priority;
  int32_t mem_sync_domain;
  uint8_t mem_sync_map_default;
  uint8_t mem_sync_map_remote;
  uint8_t attr_query_available;
  uint8_t pad;
  uint32_t preferred_carveout;
} fdy_common_attrs;

typedef struct fdy_generator {
  uint64_t id;
  uint64_t seed;
  uint64_t wholegraph_increment;
} fdy_generator;

typedef struct fdy_dep {
  uint32_t from;
  uint32_t to;
} fdy_dep;

#pragma pack(pop)

/* Memory types that mark a memcpy endpoint as device-addressable
 * (CU_MEMORYTYPE_DEVICE / CU_MEMORYTYPE_UNIFIED numbering, as stored). */
#define FDY_MEMTYPE_DEVICE 2
#define FDY_MEMTYPE_UNIFIED 4

/* Byte offsets inside a 168-B node entry that device code reads directly. */
#define FDY_NODE_OFF_TYPE 4
#define FDY_NODE_OFF_BODY 8
#define FDY_KOFF_BLOCK 8
#define FDY_KOFF_GRID 20
#define FDY_KOFF_SHMEM 32
#define FDY_KOFF_BINARY_HASH 36
#define FDY_KOFF_NAME_OFFSET 44
#define FDY_KOFF_NAME_LENGTH 48
#define FDY_KOFF_FUNC_ATTRS 52
#define FDY_KOFF_REQ_CLUSTER 64
#define FDY_KOFF_KNA_FLAGS 76
#define FDY_KOFF_KNA_CLUSTER 80
#define FDY_KOFF_KNA_END 128
#define FDY_KOFF_PARAM_INDEX 128
#define FDY_KOFF_NUM_PARAMS 132
#define FDY_KOFF_ARG_OFFSET 136
#define FDY_KOFF_ARG_SIZE 140
#define FDY_MSOFF_DST 8
#define FDY_MCOFF_DST 32
#define FDY_MCOFF_DST_MEMTYPE 88
#define FDY_MCOFF_SRC 96
#define FDY_MCOFF_SRC_MEMTYPE 152
#define FDY_EVOFF_ID 8

#ifdef __cplusplus
} /* extern "C" */

static_assert(sizeof(fdy_file_header) == 64, "header is 64 B");
static_assert(sizeof(fdy_section) == 24, "section entry is 24 B");
static_assert(sizeof(fdy_kernel_body) == 136, "kernel body is 136 B");
static_assert(sizeof(fdy_memset_body) == 48, "memset body is 48 B");
static_assert(sizeof(fdy_memcpy_body) == 152, "memcpy body is 152 B");
static_assert(sizeof(fdy_node) == 168, "node entry is 168 B");
static_assert(sizeof(fdy_param) == 8, "param entry is 8 B");
static_assert(sizeof(fdy_common_attrs) == 52, "common attrs are 52 B");
static_assert(sizeof(fdy_generator) == 24, "generator entry is 24 B");
static_assert(sizeof(fdy_dep) == 8, "dependency entry is 8 B");
static_assert(__builtin_offsetof(fdy_node, u) + __builtin_offsetof(fdy_kernel_body, binary_hash) ==
                  FDY_KOFF_BINARY_HASH,
              "binary_hash offset");
static_assert(__builtin_offsetof(fdy_node, u) + __builtin_offsetof(fdy_kernel_body, kna_flags) ==
                  FDY_KOFF_KNA_FLAGS,
              "kna_flags offset");
static_assert(__builtin_offsetof(fdy_node, u) + __builtin_offsetof(fdy_kernel_body, param_index_offset) ==
                  FDY_KOFF_PARAM_INDEX,
              "param_index_offset offset");
static_assert(__builtin_offsetof(fdy_node, u) + __builtin_offsetof(fdy_memcpy_body, src) == FDY_MCOFF_SRC,
              "memcpy src offset");
static_assert(__builtin_offsetof(fdy_node, u) + __builtin_offsetof(fdy_memcpy_body, src_mem_type) ==
                  FDY_MCOFF_SRC_MEMTYPE,
              "memcpy src type offset");
#endif

#endif /* FDY_FORMAT_H */
