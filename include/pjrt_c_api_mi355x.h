/*
 * pjrt_c_api_mi355x.h -- the PJRT C API types this plugin's GetPjrtApi table
 * uses, restated for API 0.114 (the version the reference pins:
 * /root/reference/README.md:86-96 "XLA / PJRT header dcf304bc", and
 * tests/test_pjrt_client_ownership.py:39 static_assert(PJRT_API_MINOR == 114)).
 *
 * The reference compiles against XLA's xla/pjrt/c/pjrt_c_api.h, fetched by
 * its setup script; that header is not in the reference tree or in this
 * image, and no jaxlib is installed here to check a layout against.  This
 * file is this project's own statement of the public C API:
 *   - the order of the PJRT_Api function table follows the reference's
 *     table (src/pjrt_plugin/api/pjrt_api.cc:160-321, a C++20 designated
 *     initializer, which must name members in declaration order);
 *   - the error and memory function tables follow the reference's
 *     positional initializers (api/pjrt_memory.cc:24-31, :102-104);
 *   - every argument struct lists the fields the reference's callbacks read
 *     and write (api/pjrt_*.cc), each struct starting with struct_size and
 *     extension_start as every PJRT argument struct does.
 * The plugin checks args->struct_size against the sizes below before
 * touching a field, so a caller built against a shorter struct is served
 * from the prefix it has.  Fields of API versions after 0.102 that the
 * reference leaves null are not listed; the table ends with the 0.102
 * member PJRT_Executable_ParameterMemoryKinds.
 */
#ifndef PJRT_C_API_MI355X_H_
#define PJRT_C_API_MI355X_H_

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PJRT_API_MAJOR 0
#define PJRT_API_MINOR 114

/* Size of a struct up to and including `last_field`. */
#define PJRT_STRUCT_SIZE(sname, last_field) (offsetof(sname, last_field) + sizeof(((sname*)0)->last_field))

#define PJRT_DEFINE_STRUCT_TRAITS(sname, last_field) \
  typedef struct sname sname;                         \
  enum { sname##_STRUCT_SIZE = PJRT_STRUCT_SIZE(sname, last_field) }

typedef enum {
  PJRT_Extension_Type_Gpu_Custom_Call = 0,
  PJRT_Extension_Type_Profiler,
  PJRT_Extension_Type_Custom_Partitioner,
  PJRT_Extension_Type_Stream,
  PJRT_Extension_Type_Layouts,
  PJRT_Extension_Type_FFI,
  PJRT_Extension_Type_MemoryDescriptions
} PJRT_Extension_Type;

typedef struct PJRT_Extension_Base {
  size_t struct_size;
  PJRT_Extension_Type type;
  struct PJRT_Extension_Base* next;
} PJRT_Extension_Base;

#define PJRT_ARGS_PREFIX     \
  size_t struct_size;        \
  PJRT_Extension_Base* extension_start

/* ---------------------------------------------------------------- handles */
typedef struct PJRT_Client PJRT_Client;
typedef struct PJRT_Device PJRT_Device;
typedef struct PJRT_DeviceDescription PJRT_DeviceDescription;
typedef struct PJRT_TopologyDescription PJRT_TopologyDescription;
typedef struct PJRT_Executable PJRT_Executable;
typedef struct PJRT_LoadedExecutable PJRT_LoadedExecutable;
typedef struct PJRT_Buffer PJRT_Buffer;
typedef struct PJRT_Event PJRT_Event;
typedef struct PJRT_CopyToDeviceStream PJRT_CopyToDeviceStream;
typedef struct PJRT_SerializedExecutable PJRT_SerializedExecutable;
typedef struct PJRT_SerializedTopology PJRT_SerializedTopology;
typedef struct PJRT_DeviceAssignmentSerialized PJRT_DeviceAssignmentSerialized;
typedef struct PJRT_ExecuteContext PJRT_ExecuteContext;

typedef enum {
  PJRT_Error_Code_OK = 0,
  PJRT_Error_Code_CANCELLED = 1,
  PJRT_Error_Code_UNKNOWN = 2,
  PJRT_Error_Code_INVALID_ARGUMENT = 3,
  PJRT_Error_Code_DEADLINE_EXCEEDED = 4,
  PJRT_Error_Code_NOT_FOUND = 5,
  PJRT_Error_Code_ALREADY_EXISTS = 6,
  PJRT_Error_Code_PERMISSION_DENIED = 7,
  PJRT_Error_Code_RESOURCE_EXHAUSTED = 8,
  PJRT_Error_Code_FAILED_PRECONDITION = 9,
  PJRT_Error_Code_ABORTED = 10,
  PJRT_Error_Code_OUT_OF_RANGE = 11,
  PJRT_Error_Code_UNIMPLEMENTED = 12,
  PJRT_Error_Code_INTERNAL = 13,
  PJRT_Error_Code_UNAVAILABLE = 14,
  PJRT_Error_Code_DATA_LOSS = 15,
  PJRT_Error_Code_UNAUTHENTICATED = 16
} PJRT_Error_Code;

/* Errors carry a static function table from API 0.107 (the reference's
 * pjrt_handles.h:25-33 completes the opaque base only before 0.107). */
typedef struct PJRT_Error PJRT_Error;
typedef void (*PJRT_Error_PayloadVisitor)(const char* key, size_t key_size, const char* value, size_t value_size,
                                          void* user_arg);
typedef struct PJRT_Error_FunctionTable {
  size_t struct_size;
  size_t error_struct_size;
  PJRT_Extension_Base* extension_start;
  void (*destroy)(PJRT_Error* error);
  void (*message)(const PJRT_Error* error, const char** message, size_t* message_size);
  PJRT_Error_Code (*get_code)(const PJRT_Error* error);
  void (*for_each_payload)(const PJRT_Error* error, PJRT_Error_PayloadVisitor visitor, void* user_arg);
} PJRT_Error_FunctionTable;
enum { PJRT_Error_FunctionTable_STRUCT_SIZE = PJRT_STRUCT_SIZE(PJRT_Error_FunctionTable, for_each_payload) };
struct PJRT_Error {
  const PJRT_Error_FunctionTable* vtable;
};
enum { PJRT_Error_STRUCT_SIZE = PJRT_STRUCT_SIZE(PJRT_Error, vtable) };

/* Memories carry a user-data function table from API 0.105
 * (pjrt_handles.h:25-27, pjrt_memory.cc:99-105). */
typedef struct PJRT_Memory PJRT_Memory;
typedef struct PJRT_Memory_FunctionTable {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  size_t memory_struct_size;
  void* (*get_user_data)(PJRT_Memory* memory, const void* key);
  void (*set_user_data)(PJRT_Memory* memory, const void* key, void* data, void (*dtor)(void*));
} PJRT_Memory_FunctionTable;
enum { PJRT_Memory_FunctionTable_STRUCT_SIZE = PJRT_STRUCT_SIZE(PJRT_Memory_FunctionTable, set_user_data) };
struct PJRT_Memory {
  const PJRT_Memory_FunctionTable* vtable;
};
enum { PJRT_Memory_STRUCT_SIZE = PJRT_STRUCT_SIZE(PJRT_Memory, vtable) };

/* ------------------------------------------------------------ api version */
struct PJRT_Api_Version {
  PJRT_ARGS_PREFIX;
  int major_version;
  int minor_version;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Api_Version, minor_version);

/* ----------------------------------------------------------------- errors */
struct PJRT_Error_Destroy_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Error* error;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Error_Destroy_Args, error);

struct PJRT_Error_Message_Args {
  PJRT_ARGS_PREFIX;
  const PJRT_Error* error;
  const char* message;
  size_t message_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Error_Message_Args, message_size);

struct PJRT_Error_GetCode_Args {
  PJRT_ARGS_PREFIX;
  const PJRT_Error* error;
  PJRT_Error_Code code;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Error_GetCode_Args, code);

struct PJRT_Error_ForEachPayload_Args {
  PJRT_ARGS_PREFIX;
  const PJRT_Error* error;
  PJRT_Error_PayloadVisitor visitor;
  void* user_arg;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Error_ForEachPayload_Args, user_arg);

/* ------------------------------------------------------------ named values */
typedef enum {
  PJRT_NamedValue_kString = 0,
  PJRT_NamedValue_kInt64,
  PJRT_NamedValue_kInt64List,
  PJRT_NamedValue_kFloat,
  PJRT_NamedValue_kBool
} PJRT_NamedValue_Type;

struct PJRT_NamedValue {
  PJRT_ARGS_PREFIX;
  const char* name;
  size_t name_size;
  PJRT_NamedValue_Type type;
  union {
    const char* string_value;
    int64_t int64_value;
    const int64_t* int64_array_value;
    float float_value;
    bool bool_value;
  };
  size_t value_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_NamedValue, value_size);

/* ----------------------------------------------------------------- plugin */
struct PJRT_Plugin_Initialize_Args {
  PJRT_ARGS_PREFIX;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Plugin_Initialize_Args, extension_start);

struct PJRT_Plugin_Attributes_Args {
  PJRT_ARGS_PREFIX;
  const PJRT_NamedValue* attributes;
  size_t num_attributes;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Plugin_Attributes_Args, num_attributes);

/* ----------------------------------------------------------------- events */
struct PJRT_Event_Destroy_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Event* event;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Event_Destroy_Args, event);

struct PJRT_Event_IsReady_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Event* event;
  bool is_ready;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Event_IsReady_Args, is_ready);

struct PJRT_Event_Error_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Event* event;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Event_Error_Args, event);

struct PJRT_Event_Await_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Event* event;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Event_Await_Args, event);

typedef void (*PJRT_Event_OnReadyCallback)(PJRT_Error* error, void* user_arg);
struct PJRT_Event_OnReady_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Event* event;
  PJRT_Event_OnReadyCallback callback;
  void* user_arg;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Event_OnReady_Args, user_arg);

struct PJRT_Event_Create_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Event* event;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Event_Create_Args, event);

struct PJRT_Event_Set_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Event* event;
  PJRT_Error_Code error_code;
  const char* error_message;
  size_t error_message_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Event_Set_Args, error_message_size);

/* ------------------------------------------------------------ buffer types */
typedef enum {
  PJRT_Buffer_Type_INVALID = 0,
  PJRT_Buffer_Type_PRED,
  PJRT_Buffer_Type_S8,
  PJRT_Buffer_Type_S16,
  PJRT_Buffer_Type_S32,
  PJRT_Buffer_Type_S64,
  PJRT_Buffer_Type_U8,
  PJRT_Buffer_Type_U16,
  PJRT_Buffer_Type_U32,
  PJRT_Buffer_Type_U64,
  PJRT_Buffer_Type_F16,
  PJRT_Buffer_Type_F32,
  PJRT_Buffer_Type_F64,
  PJRT_Buffer_Type_BF16
} PJRT_Buffer_Type;

typedef enum {
  PJRT_HostBufferSemantics_kImmutableOnlyDuringCall = 0,
  PJRT_HostBufferSemantics_kImmutableUntilTransferCompletes,
  PJRT_HostBufferSemantics_kImmutableZeroCopy,
  PJRT_HostBufferSemantics_kMutableZeroCopy
} PJRT_HostBufferSemantics;

typedef enum {
  PJRT_Buffer_MemoryLayout_Type_Tiled = 0,
  PJRT_Buffer_MemoryLayout_Type_Strides
} PJRT_Buffer_MemoryLayout_Type;

struct PJRT_Buffer_MemoryLayout_Tiled {
  PJRT_ARGS_PREFIX;
  const int64_t* minor_to_major;
  size_t minor_to_major_size;
  const int64_t* tile_dims;
  const size_t* tile_dim_sizes;
  size_t num_tiles;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_MemoryLayout_Tiled, num_tiles);

struct PJRT_Buffer_MemoryLayout_Strides {
  PJRT_ARGS_PREFIX;
  const int64_t* byte_strides;
  size_t num_byte_strides;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_MemoryLayout_Strides, num_byte_strides);

struct PJRT_Buffer_MemoryLayout {
  PJRT_ARGS_PREFIX;
  union {
    PJRT_Buffer_MemoryLayout_Tiled tiled;
    PJRT_Buffer_MemoryLayout_Strides strides;
  };
  PJRT_Buffer_MemoryLayout_Type type;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_MemoryLayout, type);

/* ----------------------------------------------------------------- client */
struct PJRT_KeyValueGetCallback_Args;
struct PJRT_KeyValuePutCallback_Args;
typedef PJRT_Error* (*PJRT_KeyValueGetCallback)(struct PJRT_KeyValueGetCallback_Args* args);
typedef PJRT_Error* (*PJRT_KeyValuePutCallback)(struct PJRT_KeyValuePutCallback_Args* args);

struct PJRT_Client_Create_Args {
  PJRT_ARGS_PREFIX;
  const PJRT_NamedValue* create_options;
  size_t num_options;
  PJRT_KeyValueGetCallback kv_get_callback;
  void* kv_get_user_arg;
  PJRT_KeyValuePutCallback kv_put_callback;
  void* kv_put_user_arg;
  PJRT_Client* client; /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_Create_Args, client);

struct PJRT_Client_Destroy_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_Destroy_Args, client);

struct PJRT_Client_PlatformName_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  const char* platform_name;
  size_t platform_name_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_PlatformName_Args, platform_name_size);

struct PJRT_Client_ProcessIndex_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  int process_index;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_ProcessIndex_Args, process_index);

struct PJRT_Client_PlatformVersion_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  const char* platform_version;
  size_t platform_version_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_PlatformVersion_Args, platform_version_size);

struct PJRT_Client_TopologyDescription_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  PJRT_TopologyDescription* topology;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_TopologyDescription_Args, topology);

struct PJRT_Client_Devices_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  PJRT_Device* const* devices;
  size_t num_devices;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_Devices_Args, num_devices);

struct PJRT_Client_AddressableDevices_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  PJRT_Device* const* addressable_devices;
  size_t num_addressable_devices;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_AddressableDevices_Args, num_addressable_devices);

struct PJRT_Client_LookupDevice_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  int id;
  PJRT_Device* device;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_LookupDevice_Args, device);

struct PJRT_Client_LookupAddressableDevice_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  int local_hardware_id;
  PJRT_Device* addressable_device;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_LookupAddressableDevice_Args, addressable_device);

struct PJRT_Client_AddressableMemories_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  PJRT_Memory* const* addressable_memories;
  size_t num_addressable_memories;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_AddressableMemories_Args, num_addressable_memories);

struct PJRT_Program {
  PJRT_ARGS_PREFIX;
  char* code;
  size_t code_size;
  const char* format;
  size_t format_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Program, format_size);

struct PJRT_Client_Compile_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  const PJRT_Program* program;
  const char* compile_options;
  size_t compile_options_size;
  PJRT_LoadedExecutable* executable; /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_Compile_Args, executable);

struct PJRT_Client_DefaultDeviceAssignment_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  int num_replicas;
  int num_partitions;
  size_t default_assignment_size;
  int* default_assignment; /* caller-allocated, num_replicas * num_partitions */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_DefaultDeviceAssignment_Args, default_assignment);

struct PJRT_Client_BufferFromHostBuffer_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  const void* data;
  PJRT_Buffer_Type type;
  const int64_t* dims;
  size_t num_dims;
  const int64_t* byte_strides;
  size_t num_byte_strides;
  PJRT_HostBufferSemantics host_buffer_semantics;
  PJRT_Device* device;
  PJRT_Memory* memory;
  PJRT_Buffer_MemoryLayout* device_layout;
  PJRT_Event* done_with_host_buffer; /* out */
  PJRT_Buffer* buffer;               /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_BufferFromHostBuffer_Args, buffer);

struct PJRT_Client_CreateViewOfDeviceBuffer_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  void* device_buffer_ptr;
  const int64_t* dims;
  size_t num_dims;
  PJRT_Buffer_Type element_type;
  PJRT_Buffer_MemoryLayout* layout;
  PJRT_Device* device;
  void (*on_delete_callback)(void* device_buffer_ptr, void* user_arg);
  void* on_delete_callback_arg;
  intptr_t stream;
  PJRT_Buffer* buffer; /* out */
  PJRT_Memory* memory;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_CreateViewOfDeviceBuffer_Args, memory);

struct PJRT_Client_CreateUninitializedBuffer_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  const int64_t* shape_dims;
  size_t shape_num_dims;
  PJRT_Buffer_Type shape_element_type;
  PJRT_Buffer_MemoryLayout* shape_layout;
  PJRT_Device* device;
  PJRT_Memory* memory;
  PJRT_Buffer* buffer; /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_CreateUninitializedBuffer_Args, buffer);

struct PJRT_Client_CreateErrorBuffer_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  PJRT_Error_Code error_code;
  const char* error_message;
  size_t error_message_size;
  const int64_t* shape_dims;
  size_t shape_num_dims;
  PJRT_Buffer_Type shape_element_type;
  PJRT_Buffer_MemoryLayout* shape_layout;
  PJRT_Memory* memory;
  PJRT_Buffer* buffer; /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Client_CreateErrorBuffer_Args, buffer);

/* ------------------------------------------------------- device metadata */
struct PJRT_DeviceDescription_Id_Args {
  PJRT_ARGS_PREFIX;
  PJRT_DeviceDescription* device_description;
  int id;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_DeviceDescription_Id_Args, id);

struct PJRT_DeviceDescription_ProcessIndex_Args {
  PJRT_ARGS_PREFIX;
  PJRT_DeviceDescription* device_description;
  int process_index;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_DeviceDescription_ProcessIndex_Args, process_index);

struct PJRT_DeviceDescription_Attributes_Args {
  PJRT_ARGS_PREFIX;
  PJRT_DeviceDescription* device_description;
  size_t num_attributes;
  const PJRT_NamedValue* attributes;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_DeviceDescription_Attributes_Args, attributes);

struct PJRT_DeviceDescription_Kind_Args {
  PJRT_ARGS_PREFIX;
  PJRT_DeviceDescription* device_description;
  const char* device_kind;
  size_t device_kind_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_DeviceDescription_Kind_Args, device_kind_size);

struct PJRT_DeviceDescription_DebugString_Args {
  PJRT_ARGS_PREFIX;
  PJRT_DeviceDescription* device_description;
  const char* debug_string;
  size_t debug_string_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_DeviceDescription_DebugString_Args, debug_string_size);

struct PJRT_DeviceDescription_ToString_Args {
  PJRT_ARGS_PREFIX;
  PJRT_DeviceDescription* device_description;
  const char* to_string;
  size_t to_string_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_DeviceDescription_ToString_Args, to_string_size);

struct PJRT_Device_GetDescription_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Device* device;
  PJRT_DeviceDescription* device_description;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Device_GetDescription_Args, device_description);

struct PJRT_Device_IsAddressable_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Device* device;
  bool is_addressable;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Device_IsAddressable_Args, is_addressable);

struct PJRT_Device_LocalHardwareId_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Device* device;
  int local_hardware_id;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Device_LocalHardwareId_Args, local_hardware_id);

struct PJRT_Device_AddressableMemories_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Device* device;
  PJRT_Memory* const* memories;
  size_t num_memories;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Device_AddressableMemories_Args, num_memories);

struct PJRT_Device_DefaultMemory_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Device* device;
  PJRT_Memory* memory;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Device_DefaultMemory_Args, memory);

/* The 0.114 header appends peak_allocated_bytes(_is_set); the reference
 * fills them only when the caller's struct_size covers them
 * (api/pjrt_device.cc:131-137). */
struct PJRT_Device_MemoryStats_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Device* device;
  int64_t bytes_in_use;
  int64_t peak_bytes_in_use;
  bool peak_bytes_in_use_is_set;
  int64_t num_allocs;
  bool num_allocs_is_set;
  int64_t largest_alloc_size;
  bool largest_alloc_size_is_set;
  int64_t bytes_limit;
  bool bytes_limit_is_set;
  int64_t bytes_reserved;
  bool bytes_reserved_is_set;
  int64_t peak_bytes_reserved;
  bool peak_bytes_reserved_is_set;
  int64_t bytes_reservable_limit;
  bool bytes_reservable_limit_is_set;
  int64_t largest_free_block_bytes;
  bool largest_free_block_bytes_is_set;
  int64_t pool_bytes;
  bool pool_bytes_is_set;
  int64_t peak_pool_bytes;
  bool peak_pool_bytes_is_set;
  int64_t peak_allocated_bytes;
  bool peak_allocated_bytes_is_set;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Device_MemoryStats_Args, peak_allocated_bytes_is_set);

/* ----------------------------------------------------------------- memory */
struct PJRT_Memory_Id_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Memory* memory;
  int id;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Memory_Id_Args, id);

struct PJRT_Memory_Kind_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Memory* memory;
  const char* kind;
  size_t kind_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Memory_Kind_Args, kind_size);

struct PJRT_Memory_Kind_Id_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Memory* memory;
  int kind_id;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Memory_Kind_Id_Args, kind_id);

struct PJRT_Memory_DebugString_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Memory* memory;
  const char* debug_string;
  size_t debug_string_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Memory_DebugString_Args, debug_string_size);

struct PJRT_Memory_ToString_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Memory* memory;
  const char* to_string;
  size_t to_string_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Memory_ToString_Args, to_string_size);

struct PJRT_Memory_AddressableByDevices_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Memory* memory;
  PJRT_Device* const* devices;
  size_t num_devices;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Memory_AddressableByDevices_Args, num_devices);

/* ------------------------------------------------------------- executable */
struct PJRT_Executable_Destroy_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Executable* executable;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_Destroy_Args, executable);

struct PJRT_LoadedExecutable_Destroy_Args {
  PJRT_ARGS_PREFIX;
  PJRT_LoadedExecutable* executable;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_LoadedExecutable_Destroy_Args, executable);

struct PJRT_LoadedExecutable_GetExecutable_Args {
  PJRT_ARGS_PREFIX;
  PJRT_LoadedExecutable* loaded_executable;
  PJRT_Executable* executable; /* out, owned by the caller */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_LoadedExecutable_GetExecutable_Args, executable);

struct PJRT_Executable_Name_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Executable* executable;
  const char* executable_name;
  size_t executable_name_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_Name_Args, executable_name_size);

struct PJRT_Executable_NumReplicas_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Executable* executable;
  size_t num_replicas;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_NumReplicas_Args, num_replicas);

struct PJRT_Executable_NumPartitions_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Executable* executable;
  size_t num_partitions;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_NumPartitions_Args, num_partitions);

struct PJRT_LoadedExecutable_AddressableDevices_Args {
  PJRT_ARGS_PREFIX;
  PJRT_LoadedExecutable* executable;
  PJRT_Device* const* addressable_devices;
  size_t num_addressable_devices;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_LoadedExecutable_AddressableDevices_Args, num_addressable_devices);

struct PJRT_Executable_OptimizedProgram_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Executable* executable;
  PJRT_Program* program; /* in/out: code == NULL asks for the size */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_OptimizedProgram_Args, program);

struct PJRT_LoadedExecutable_Delete_Args {
  PJRT_ARGS_PREFIX;
  PJRT_LoadedExecutable* executable;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_LoadedExecutable_Delete_Args, executable);

struct PJRT_LoadedExecutable_IsDeleted_Args {
  PJRT_ARGS_PREFIX;
  PJRT_LoadedExecutable* executable;
  bool is_deleted;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_LoadedExecutable_IsDeleted_Args, is_deleted);

typedef struct PJRT_Chunk {
  void* data;
  size_t size;
  void (*deleter)(void* data, void* deleter_arg);
  void* deleter_arg;
} PJRT_Chunk;

typedef struct PJRT_CallbackError PJRT_CallbackError;
typedef PJRT_Error* (*PJRT_SendCallback)(PJRT_Chunk* chunk, PJRT_CallbackError* callback_error,
                                         size_t total_size_in_bytes, bool done, void* user_arg);
typedef void (*PJRT_RecvCallback)(PJRT_CopyToDeviceStream* stream, void* user_arg);

typedef struct PJRT_SendCallbackInfo {
  int64_t channel_id;
  void* user_arg;
  PJRT_SendCallback send_callback;
} PJRT_SendCallbackInfo;

typedef struct PJRT_RecvCallbackInfo {
  int64_t channel_id;
  void* user_arg;
  PJRT_RecvCallback recv_callback;
} PJRT_RecvCallbackInfo;

struct PJRT_ExecuteOptions {
  PJRT_ARGS_PREFIX;
  PJRT_SendCallbackInfo** send_callbacks;
  PJRT_RecvCallbackInfo** recv_callbacks;
  size_t num_send_ops;
  size_t num_recv_ops;
  int launch_id;
  const int64_t* non_donatable_input_indices;
  size_t num_non_donatable_input_indices;
  PJRT_ExecuteContext* context;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_ExecuteOptions, context);

struct PJRT_LoadedExecutable_Execute_Args {
  PJRT_ARGS_PREFIX;
  PJRT_LoadedExecutable* executable;
  PJRT_ExecuteOptions* options;
  PJRT_Buffer* const* const* argument_lists; /* [num_devices][num_args] */
  size_t num_devices;
  size_t num_args;
  PJRT_Buffer** const* output_lists;   /* [num_devices][num_outputs], filled */
  PJRT_Event** device_complete_events; /* [num_devices] or NULL */
  PJRT_Device* execute_device;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_LoadedExecutable_Execute_Args, execute_device);

struct PJRT_Executable_NumOutputs_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Executable* executable;
  size_t num_outputs;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_NumOutputs_Args, num_outputs);

struct PJRT_Executable_SizeOfGeneratedCodeInBytes_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Executable* executable;
  int64_t size_in_bytes;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args, size_in_bytes);

struct PJRT_Executable_Fingerprint_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Executable* executable;
  const char* executable_fingerprint;
  size_t executable_fingerprint_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_Fingerprint_Args, executable_fingerprint_size);

struct PJRT_Executable_GetCostAnalysis_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Executable* executable;
  size_t num_properties;
  const PJRT_NamedValue* properties;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_GetCostAnalysis_Args, properties);

struct PJRT_Executable_OutputElementTypes_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Executable* executable;
  PJRT_Buffer_Type* output_types;
  size_t num_output_types;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_OutputElementTypes_Args, num_output_types);

struct PJRT_Executable_OutputDimensions_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Executable* executable;
  size_t num_outputs;
  const int64_t* dims;     /* all outputs' dims, concatenated */
  const size_t* dim_sizes; /* rank of each output */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_OutputDimensions_Args, dim_sizes);

struct PJRT_Executable_OutputMemoryKinds_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Executable* executable;
  size_t num_outputs;
  const char* const* memory_kinds;
  const size_t* memory_kind_sizes;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_OutputMemoryKinds_Args, memory_kind_sizes);

struct PJRT_Executable_ParameterMemoryKinds_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Executable* executable;
  size_t num_parameters;
  const char* const* memory_kinds;
  const size_t* memory_kind_sizes;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_ParameterMemoryKinds_Args, memory_kind_sizes);

struct PJRT_Executable_Serialize_Args {
  PJRT_ARGS_PREFIX;
  const PJRT_Executable* executable;
  const char* serialized_bytes;
  size_t serialized_bytes_size;
  PJRT_SerializedExecutable* serialized_executable;
  void (*serialized_executable_deleter)(PJRT_SerializedExecutable* exec);
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_Serialize_Args, serialized_executable_deleter);

struct PJRT_Executable_DeserializeAndLoad_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Client* client;
  const char* serialized_executable;
  size_t serialized_executable_size;
  PJRT_LoadedExecutable* loaded_executable; /* out */
  const char* overridden_serialized_compile_options;
  size_t overridden_serialized_compile_options_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Executable_DeserializeAndLoad_Args, overridden_serialized_compile_options_size);

struct PJRT_LoadedExecutable_Fingerprint_Args {
  PJRT_ARGS_PREFIX;
  PJRT_LoadedExecutable* executable;
  const char* executable_fingerprint;
  size_t executable_fingerprint_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_LoadedExecutable_Fingerprint_Args, executable_fingerprint_size);

struct PJRT_LoadedExecutable_GetDeviceAssignment_Args {
  PJRT_ARGS_PREFIX;
  PJRT_LoadedExecutable* executable;
  const char* serialized_bytes;
  size_t serialized_bytes_size;
  PJRT_DeviceAssignmentSerialized* serialized_device_assignment;
  void (*serialized_device_assignment_deleter)(PJRT_DeviceAssignmentSerialized* da);
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_LoadedExecutable_GetDeviceAssignment_Args, serialized_device_assignment_deleter);

/* ---------------------------------------------------------------- buffers */
struct PJRT_Buffer_Destroy_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_Destroy_Args, buffer);

struct PJRT_Buffer_ElementType_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  PJRT_Buffer_Type type;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_ElementType_Args, type);

struct PJRT_Buffer_Dimensions_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  const int64_t* dims;
  size_t num_dims;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_Dimensions_Args, num_dims);

struct PJRT_Buffer_UnpaddedDimensions_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  const int64_t* unpadded_dims;
  size_t num_dims;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_UnpaddedDimensions_Args, num_dims);

struct PJRT_Buffer_DynamicDimensionIndices_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  const size_t* dynamic_dim_indices;
  size_t num_dynamic_dims;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_DynamicDimensionIndices_Args, num_dynamic_dims);

struct PJRT_Buffer_GetMemoryLayout_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  PJRT_Buffer_MemoryLayout layout; /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_GetMemoryLayout_Args, layout);

struct PJRT_Buffer_ToHostBuffer_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* src;
  PJRT_Buffer_MemoryLayout* host_layout;
  void* dst; /* NULL: report the size in dst_size */
  size_t dst_size;
  PJRT_Event* event; /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_ToHostBuffer_Args, event);

struct PJRT_Buffer_OnDeviceSizeInBytes_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  size_t on_device_size_in_bytes;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_OnDeviceSizeInBytes_Args, on_device_size_in_bytes);

struct PJRT_Buffer_Delete_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_Delete_Args, buffer);

struct PJRT_Buffer_IsDeleted_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  bool is_deleted;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_IsDeleted_Args, is_deleted);

struct PJRT_Buffer_CopyRawToHost_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  void* dst;
  int64_t offset;
  int64_t transfer_size;
  PJRT_Event* event; /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_CopyRawToHost_Args, event);

struct PJRT_Buffer_CopyRawToHostFuture_Callback_Args {
  PJRT_ARGS_PREFIX;
  void* callback_data;
  PJRT_Error_Code error_code;
  const char* error_message;
  size_t error_message_size;
  void* dst;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_CopyRawToHostFuture_Callback_Args, dst);

struct PJRT_Buffer_CopyRawToHostFuture_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  int64_t offset;
  int64_t transfer_size;
  PJRT_Event* event; /* out */
  void* callback_data; /* out */
  void (*future_ready_callback)(PJRT_Buffer_CopyRawToHostFuture_Callback_Args* args); /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_CopyRawToHostFuture_Args, future_ready_callback);

struct PJRT_Buffer_CopyToDevice_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  PJRT_Device* dst_device;
  PJRT_Buffer* dst_buffer; /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_CopyToDevice_Args, dst_buffer);

struct PJRT_Buffer_CopyToMemory_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  PJRT_Memory* dst_memory;
  PJRT_Buffer* dst_buffer; /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_CopyToMemory_Args, dst_buffer);

struct PJRT_Buffer_IsOnCpu_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  bool is_on_cpu;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_IsOnCpu_Args, is_on_cpu);

struct PJRT_Buffer_Device_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  PJRT_Device* device;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_Device_Args, device);

struct PJRT_Buffer_Memory_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  PJRT_Memory* memory;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_Memory_Args, memory);

struct PJRT_Buffer_ReadyEvent_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  PJRT_Event* event; /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_ReadyEvent_Args, event);

struct PJRT_Buffer_UnsafePointer_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  uintptr_t buffer_pointer;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_UnsafePointer_Args, buffer_pointer);

struct PJRT_Buffer_IncreaseExternalReferenceCount_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_IncreaseExternalReferenceCount_Args, buffer);

struct PJRT_Buffer_DecreaseExternalReferenceCount_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_DecreaseExternalReferenceCount_Args, buffer);

struct PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args {
  PJRT_ARGS_PREFIX;
  PJRT_Buffer* buffer;
  void* device_memory_ptr;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args, device_memory_ptr);

/* ---------------------------------------------------- copy-to-device stream */
struct PJRT_CopyToDeviceStream_Destroy_Args {
  PJRT_ARGS_PREFIX;
  PJRT_CopyToDeviceStream* stream;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_CopyToDeviceStream_Destroy_Args, stream);

struct PJRT_CopyToDeviceStream_AddChunk_Args {
  PJRT_ARGS_PREFIX;
  PJRT_CopyToDeviceStream* stream;
  PJRT_Chunk* chunk;
  PJRT_Event* transfer_complete;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_CopyToDeviceStream_AddChunk_Args, transfer_complete);

struct PJRT_CopyToDeviceStream_TotalBytes_Args {
  PJRT_ARGS_PREFIX;
  PJRT_CopyToDeviceStream* stream;
  int64_t total_bytes;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_CopyToDeviceStream_TotalBytes_Args, total_bytes);

struct PJRT_CopyToDeviceStream_GranuleSize_Args {
  PJRT_ARGS_PREFIX;
  PJRT_CopyToDeviceStream* stream;
  int64_t granule_size_in_bytes;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_CopyToDeviceStream_GranuleSize_Args, granule_size_in_bytes);

struct PJRT_CopyToDeviceStream_CurrentBytes_Args {
  PJRT_ARGS_PREFIX;
  PJRT_CopyToDeviceStream* stream;
  int64_t current_bytes;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_CopyToDeviceStream_CurrentBytes_Args, current_bytes);

/* ---------------------------------------------------------------- topology */
struct PJRT_TopologyDescription_Create_Args {
  PJRT_ARGS_PREFIX;
  const char* topology_name;
  size_t topology_name_size;
  const PJRT_NamedValue* create_options;
  size_t num_options;
  PJRT_TopologyDescription* topology; /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_TopologyDescription_Create_Args, topology);

struct PJRT_TopologyDescription_Destroy_Args {
  PJRT_ARGS_PREFIX;
  PJRT_TopologyDescription* topology;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_TopologyDescription_Destroy_Args, topology);

struct PJRT_TopologyDescription_PlatformName_Args {
  PJRT_ARGS_PREFIX;
  PJRT_TopologyDescription* topology;
  const char* platform_name;
  size_t platform_name_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_TopologyDescription_PlatformName_Args, platform_name_size);

struct PJRT_TopologyDescription_PlatformVersion_Args {
  PJRT_ARGS_PREFIX;
  PJRT_TopologyDescription* topology;
  const char* platform_version;
  size_t platform_version_size;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_TopologyDescription_PlatformVersion_Args, platform_version_size);

struct PJRT_TopologyDescription_GetDeviceDescriptions_Args {
  PJRT_ARGS_PREFIX;
  PJRT_TopologyDescription* topology;
  PJRT_DeviceDescription* const* descriptions;
  size_t num_descriptions;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_TopologyDescription_GetDeviceDescriptions_Args, num_descriptions);

struct PJRT_TopologyDescription_Serialize_Args {
  PJRT_ARGS_PREFIX;
  PJRT_TopologyDescription* topology;
  const char* serialized_bytes;
  size_t serialized_bytes_size;
  PJRT_SerializedTopology* serialized_topology;
  void (*serialized_topology_deleter)(PJRT_SerializedTopology* serialized_topology);
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_TopologyDescription_Serialize_Args, serialized_topology_deleter);

struct PJRT_TopologyDescription_Attributes_Args {
  PJRT_ARGS_PREFIX;
  PJRT_TopologyDescription* topology;
  const PJRT_NamedValue* attributes;
  size_t num_attributes;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_TopologyDescription_Attributes_Args, num_attributes);

struct PJRT_TopologyDescription_Fingerprint_Args {
  PJRT_ARGS_PREFIX;
  PJRT_TopologyDescription* topology;
  uint64_t fingerprint;
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_TopologyDescription_Fingerprint_Args, fingerprint);

struct PJRT_Compile_Args {
  PJRT_ARGS_PREFIX;
  const PJRT_TopologyDescription* topology;
  const PJRT_Program* program;
  const char* compile_options;
  size_t compile_options_size;
  PJRT_Client* client;
  PJRT_Executable* executable; /* out */
};
PJRT_DEFINE_STRUCT_TRAITS(PJRT_Compile_Args, executable);

/* ------------------------------------------------------------- the table */
#define PJRT_API_FN(name) PJRT_Error* (*name)(struct name##_Args * args)
/* Entries this plugin leaves NULL (the reference leaves them NULL too,
 * api/pjrt_api.cc:281-310) are typed as opaque function pointers. */
#define PJRT_API_UNUSED(name) void* name

typedef struct PJRT_Api {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Api_Version pjrt_api_version;

  void (*PJRT_Error_Destroy)(PJRT_Error_Destroy_Args* args);
  void (*PJRT_Error_Message)(PJRT_Error_Message_Args* args);
  PJRT_API_FN(PJRT_Error_GetCode);

  PJRT_API_FN(PJRT_Plugin_Initialize);
  PJRT_API_FN(PJRT_Plugin_Attributes);

  PJRT_API_FN(PJRT_Event_Destroy);
  PJRT_API_FN(PJRT_Event_IsReady);
  PJRT_API_FN(PJRT_Event_Error);
  PJRT_API_FN(PJRT_Event_Await);
  PJRT_API_FN(PJRT_Event_OnReady);

  PJRT_API_FN(PJRT_Client_Create);
  PJRT_API_FN(PJRT_Client_Destroy);
  PJRT_API_FN(PJRT_Client_PlatformName);
  PJRT_API_FN(PJRT_Client_ProcessIndex);
  PJRT_API_FN(PJRT_Client_PlatformVersion);
  PJRT_API_FN(PJRT_Client_Devices);
  PJRT_API_FN(PJRT_Client_AddressableDevices);
  PJRT_API_FN(PJRT_Client_LookupDevice);
  PJRT_API_FN(PJRT_Client_LookupAddressableDevice);
  PJRT_API_FN(PJRT_Client_AddressableMemories);
  PJRT_API_FN(PJRT_Client_Compile);
  PJRT_API_FN(PJRT_Client_DefaultDeviceAssignment);
  PJRT_API_FN(PJRT_Client_BufferFromHostBuffer);

  PJRT_API_FN(PJRT_DeviceDescription_Id);
  PJRT_API_FN(PJRT_DeviceDescription_ProcessIndex);
  PJRT_API_FN(PJRT_DeviceDescription_Attributes);
  PJRT_API_FN(PJRT_DeviceDescription_Kind);
  PJRT_API_FN(PJRT_DeviceDescription_DebugString);
  PJRT_API_FN(PJRT_DeviceDescription_ToString);

  PJRT_API_FN(PJRT_Device_GetDescription);
  PJRT_API_FN(PJRT_Device_IsAddressable);
  PJRT_API_FN(PJRT_Device_LocalHardwareId);
  PJRT_API_FN(PJRT_Device_AddressableMemories);
  PJRT_API_FN(PJRT_Device_DefaultMemory);
  PJRT_API_FN(PJRT_Device_MemoryStats);

  PJRT_API_FN(PJRT_Memory_Id);
  PJRT_API_FN(PJRT_Memory_Kind);
  PJRT_API_FN(PJRT_Memory_DebugString);
  PJRT_API_FN(PJRT_Memory_ToString);
  PJRT_API_FN(PJRT_Memory_AddressableByDevices);

  PJRT_API_FN(PJRT_Executable_Destroy);
  PJRT_API_FN(PJRT_Executable_Name);
  PJRT_API_FN(PJRT_Executable_NumReplicas);
  PJRT_API_FN(PJRT_Executable_NumPartitions);
  PJRT_API_FN(PJRT_Executable_NumOutputs);
  PJRT_API_FN(PJRT_Executable_SizeOfGeneratedCodeInBytes);
  PJRT_API_FN(PJRT_Executable_GetCostAnalysis);
  PJRT_API_FN(PJRT_Executable_OutputMemoryKinds);
  PJRT_API_FN(PJRT_Executable_OptimizedProgram);
  PJRT_API_FN(PJRT_Executable_Serialize);

  PJRT_API_FN(PJRT_LoadedExecutable_Destroy);
  PJRT_API_FN(PJRT_LoadedExecutable_GetExecutable);
  PJRT_API_FN(PJRT_LoadedExecutable_AddressableDevices);
  PJRT_API_FN(PJRT_LoadedExecutable_Delete);
  PJRT_API_FN(PJRT_LoadedExecutable_IsDeleted);
  PJRT_API_FN(PJRT_LoadedExecutable_Execute);
  PJRT_API_FN(PJRT_Executable_DeserializeAndLoad);
  PJRT_API_FN(PJRT_LoadedExecutable_Fingerprint);

  PJRT_API_FN(PJRT_Buffer_Destroy);
  PJRT_API_FN(PJRT_Buffer_ElementType);
  PJRT_API_FN(PJRT_Buffer_Dimensions);
  PJRT_API_FN(PJRT_Buffer_UnpaddedDimensions);
  PJRT_API_FN(PJRT_Buffer_DynamicDimensionIndices);
  PJRT_API_FN(PJRT_Buffer_GetMemoryLayout);
  PJRT_API_FN(PJRT_Buffer_OnDeviceSizeInBytes);
  PJRT_API_FN(PJRT_Buffer_Device);
  PJRT_API_FN(PJRT_Buffer_Memory);
  PJRT_API_FN(PJRT_Buffer_Delete);
  PJRT_API_FN(PJRT_Buffer_IsDeleted);
  PJRT_API_FN(PJRT_Buffer_CopyToDevice);
  PJRT_API_FN(PJRT_Buffer_ToHostBuffer);
  PJRT_API_FN(PJRT_Buffer_IsOnCpu);
  PJRT_API_FN(PJRT_Buffer_ReadyEvent);
  PJRT_API_FN(PJRT_Buffer_UnsafePointer);
  PJRT_API_FN(PJRT_Buffer_IncreaseExternalReferenceCount);
  PJRT_API_FN(PJRT_Buffer_DecreaseExternalReferenceCount);
  PJRT_API_FN(PJRT_Buffer_OpaqueDeviceMemoryDataPointer);

  PJRT_API_FN(PJRT_CopyToDeviceStream_Destroy);
  PJRT_API_FN(PJRT_CopyToDeviceStream_AddChunk);
  PJRT_API_FN(PJRT_CopyToDeviceStream_TotalBytes);
  PJRT_API_FN(PJRT_CopyToDeviceStream_GranuleSize);
  PJRT_API_FN(PJRT_CopyToDeviceStream_CurrentBytes);

  PJRT_API_FN(PJRT_TopologyDescription_Create);
  PJRT_API_FN(PJRT_TopologyDescription_Destroy);
  PJRT_API_FN(PJRT_TopologyDescription_PlatformName);
  PJRT_API_FN(PJRT_TopologyDescription_PlatformVersion);
  PJRT_API_FN(PJRT_TopologyDescription_GetDeviceDescriptions);
  PJRT_API_FN(PJRT_TopologyDescription_Serialize);
  PJRT_API_FN(PJRT_TopologyDescription_Attributes);

  PJRT_API_FN(PJRT_Compile);

  PJRT_API_FN(PJRT_Executable_OutputElementTypes);
  PJRT_API_FN(PJRT_Executable_OutputDimensions);
  PJRT_API_FN(PJRT_Buffer_CopyToMemory);
  PJRT_API_FN(PJRT_Client_CreateViewOfDeviceBuffer);
  PJRT_API_FN(PJRT_Executable_Fingerprint);
  PJRT_API_FN(PJRT_Client_TopologyDescription);
  PJRT_API_UNUSED(PJRT_Executable_GetCompiledMemoryStats);
  PJRT_API_FN(PJRT_Memory_Kind_Id);
  PJRT_API_UNUSED(PJRT_ExecuteContext_Create);
  PJRT_API_UNUSED(PJRT_ExecuteContext_Destroy);
  PJRT_API_FN(PJRT_Buffer_CopyRawToHost);
  PJRT_API_UNUSED(PJRT_AsyncHostToDeviceTransferManager_Destroy);
  PJRT_API_UNUSED(PJRT_AsyncHostToDeviceTransferManager_TransferData);
  PJRT_API_UNUSED(PJRT_Client_CreateBuffersForAsyncHostToDevice);
  PJRT_API_UNUSED(PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer);
  PJRT_API_UNUSED(PJRT_AsyncHostToDeviceTransferManager_Device);
  PJRT_API_UNUSED(PJRT_AsyncHostToDeviceTransferManager_BufferCount);
  PJRT_API_UNUSED(PJRT_AsyncHostToDeviceTransferManager_BufferSize);
  PJRT_API_UNUSED(PJRT_AsyncHostToDeviceTransferManager_SetBufferError);
  PJRT_API_UNUSED(PJRT_AsyncHostToDeviceTransferManager_AddMetadata);
  PJRT_API_UNUSED(PJRT_Client_DmaMap);
  PJRT_API_UNUSED(PJRT_Client_DmaUnmap);
  PJRT_API_FN(PJRT_Client_CreateUninitializedBuffer);
  PJRT_API_UNUSED(PJRT_Client_UpdateGlobalProcessInfo);
  PJRT_API_UNUSED(PJRT_TopologyDescription_Deserialize);
  PJRT_API_UNUSED(PJRT_Client_CreateAliasBuffer);
  PJRT_API_UNUSED(PJRT_Client_FulfillAliasBuffer);
  PJRT_API_FN(PJRT_LoadedExecutable_GetDeviceAssignment);
  PJRT_API_FN(PJRT_Client_CreateErrorBuffer);
  PJRT_API_UNUSED(PJRT_AsyncHostToDeviceTransferManager_TransferLiteral);
  PJRT_API_FN(PJRT_Buffer_CopyRawToHostFuture);
  PJRT_API_UNUSED(PJRT_Device_PoisonExecution);
  PJRT_API_UNUSED(PJRT_Device_CreateAsyncTrackingEvent);
  PJRT_API_UNUSED(PJRT_AsyncTrackingEvent_Destroy);
  PJRT_API_UNUSED(PJRT_Executable_GetCompileOptions);
  PJRT_API_UNUSED(PJRT_Buffer_DonateWithControlDependency);
  PJRT_API_FN(PJRT_Event_Create);
  PJRT_API_FN(PJRT_Event_Set);
  PJRT_API_FN(PJRT_Error_ForEachPayload);
  PJRT_API_FN(PJRT_TopologyDescription_Fingerprint);
  PJRT_API_FN(PJRT_Executable_ParameterMemoryKinds);
} PJRT_Api;
enum { PJRT_Api_STRUCT_SIZE = PJRT_STRUCT_SIZE(PJRT_Api, PJRT_Executable_ParameterMemoryKinds) };

/* The one exported symbol of libmk_pjrt.so (api/pjrt_api.cc:324-329). */
const PJRT_Api* GetPjrtApi(void);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* PJRT_C_API_MI355X_H_ */
