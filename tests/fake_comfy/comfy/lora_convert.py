def convert_lora(sd):
    return sd
