// gguf.h -- the memory-mapped GGUF file reader (gguf.cpp)
#pragma once
#include <stdint.h>
#include <string.h>

#include <map>
#include <string>

#include "../../include/tie_hip.h"

namespace tie {

struct GGUFTensor {
	uint32_t n_dims = 0, type = 0;
	uint64_t ne[4] = {1, 1, 1, 1}; // ne[0] fastest (GGUF order)
	uint64_t offset = 0, bytes = 0;
	const uint8_t *data = nullptr;
};

struct GGUFFile {
	struct Meta {
		uint32_t type = 0;
		uint64_t raw = 0;
		uint64_t as_u64() const
		{
			switch (type) {
			case 0: return (uint8_t)raw;
			case 1: return (uint64_t)(int64_t)(int8_t)raw;
			case 2: return (uint16_t)raw;
			case 3: return (uint64_t)(int64_t)(int16_t)raw;
			case 4: return (uint32_t)raw;
			case 5: return (uint64_t)(int64_t)(int32_t)raw;
			case 7: return raw & 1;
			default: return raw;
			}
		}
		float as_f32() const
		{
			if (type == 6) {
				float f;
				uint32_t u = (uint32_t)raw;
				memcpy(&f, &u, 4);
				return f;
			}
			if (type == 12) {
				double x;
				memcpy(&x, &raw, 8);
				return (float)x;
			}
			return (float)as_u64();
		}
	};
	void *map = nullptr;
	size_t size = 0;
	uint64_t data_offset = 0;
	std::map<std::string, Meta> nums;
	std::map<std::string, std::string> strs;
	std::map<std::string, GGUFTensor> tensors;

	~GGUFFile();
	int open(const char *path);
	static uint64_t tensor_bytes(uint32_t type, uint64_t n);
	bool num(const std::string &key, uint64_t &v) const;
	bool f32(const std::string &key, float &v) const;
	const GGUFTensor *tensor(const std::string &name) const;
	int moe_info(tie_hip_model_info &info) const;
};

} // namespace tie
